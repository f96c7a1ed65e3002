// program.hip - ggml-compiler's runtime on this library: the GGUF program loader, its driver and
// the model C API of include/ggml_compiler_rt.h (reference: runtime/include/ggml_compiler_rt.h:91-172).
//
// A GGUF written by ggml-compiler holds weights and constants (tensors "w.N" / "c.N") and a program
// (JSON under "ggml_compiler.program", written by ggml_compiler/emit/gguf_runtime.py:104-207):
// symbols with ranges, driver values, stages whose nodes are already in ggml terms (innermost-first
// `ne`, ggml axes), entry points whose drivers call stages and run loops, and state values.
//
// Loading uploads every tensor into one HIP buffer (quantized ones in this library's packed
// layout), allocates every driver value in a second buffer (zeroed, so state starts at zero; a
// symbolic value at its largest size, viewed per binding), and builds one graph per driver call
// with the ggml API, placed by the graph allocator; each node is one ggml call, and the ggml layer
// and the backend's supports_op refuse, with the reason, what cannot run. Each entry's driver is
// compiled to flat code (calls; loops as enter / top / bottom with jumps) and run by a small
// interpreter. Everything a run does between graphs - loop carries, counters, per-iteration scalars
// and slices, causal mask rows, collected rows, the until test - is device work ordered on the
// backend's stream with the graphs; a loop reads its counters' starts once, and the host learns of
// an until stop one iteration later from a word the test op writes to host memory, so no
// iteration waits for the host (loop_bottom_device). Stage times are GPU times from events
// around each call.
//
// Semantics kept from the reference (runtime/src/ggml_compiler_rt.cpp, runtime/src/program.cpp,
// runtime/src/ops.cpp): the program schema and its checks, symbolic dims with Python's integer
// semantics, the per-iteration order of a loop (carries and counter starts at entry; then per
// iteration scalars, slices, counters, bound symbols, masks, the body, collected rows, the until
// test), results reaching driver values after every other node, the C API's argument checks and
// messages, and the GGML_COMPILER_PROFILE / GGML_COMPILER_LOG environment switches.
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
#include <cstdlib>
#include <cstring>
#include <functional>
#include <map>
#include <set>
#include <memory>
#include <unordered_map>
#include <thread>
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

// A symbolic integer dim compiled to postfix code: a literal or a symbol read pushes a value, an
// operator pops the right operand and replaces the left one. The program's n-ary form
// ["op", a, b, c] is a left fold, compiled as a b op c op. Operators follow Python on ints
// (ggml_compiler/ir/sym.py): // rounds toward minus infinity and % takes the divisor's sign.
class Dim {
  public:
    enum Op : uint8_t { Lit, Sym, Add, Mul, FloorDiv, Mod, Max, Min };
    static constexpr int kMaxDepth = 64;

    static Dim literal(int64_t v) {
        Dim d;
        d.code_.push_back({Lit, v});
        return d;
    }
    static Dim symbol(int k) {
        Dim d;
        d.code_.push_back({Sym, k});
        return d;
    }
    // this op rhs, as the next step of a left fold
    void fold(Op op, const Dim & rhs) {
        depth_ = std::max(depth_, rhs.depth_ + 1);
        if (depth_ > kMaxDepth) fail("symbolic dim nested too deeply");
        code_.insert(code_.end(), rhs.code_.begin(), rhs.code_.end());
        code_.push_back({op, 0});
    }
    bool fixed() const { return code_.size() == 1 && code_[0].op == Lit; }
    void mark(std::vector<bool> & used) const {
        for (const Insn & in : code_)
            if (in.op == Sym) used.at((size_t) in.arg) = true;
    }
    int64_t operator()(const std::vector<int64_t> & sym) const {
        int64_t st[kMaxDepth];
        int sp = 0;
        for (const Insn & in : code_) {
            if (in.op == Lit) {
                st[sp++] = in.arg;
            } else if (in.op == Sym) {
                st[sp++] = sym.at((size_t) in.arg);
            } else {
                sp--;
                st[sp - 1] = apply(in.op, st[sp - 1], st[sp]);
            }
        }
        return st[0];
    }

  private:
    struct Insn {
        Op op;
        int64_t arg;
    };
    std::vector<Insn> code_;
    int depth_ = 1;

    static int64_t apply(Op op, int64_t a, int64_t b) {
        switch (op) {
            case Add: return a + b;
            case Mul: return a * b;
            case Max: return a < b ? b : a;
            case Min: return b < a ? b : a;
            case FloorDiv:
            case Mod: {
                if (b == 0) fail(op == FloorDiv ? "division by zero in a symbolic dim" : "modulo by zero in a symbolic dim");
                lldiv_t qr = std::lldiv(a, b);  // truncating; move to the floor when the signs differ
                if (qr.rem != 0 && ((qr.rem > 0) != (b > 0))) {
                    qr.quot -= 1;
                    qr.rem += b;
                }
                return op == FloorDiv ? qr.quot : qr.rem;
            }
            default: return 0;
        }
    }
};

// A dim in the JSON: an integer, a symbol name, or [op, operand...] (ggml_compiler/ir/sym.py).
Dim parse_dim(const Json & j, const std::vector<Symbol> & syms) {
    if (j.kind == Json::Num) return Dim::literal(j.as_int());
    if (j.kind == Json::Str) {
        for (size_t k = 0; k < syms.size(); k++)
            if (syms[k].name == j.s) return Dim::symbol((int) k);
        fail("dim refers to unknown symbol '" + j.s + "'");
    }
    if (j.kind != Json::Arr || j.arr.size() < 2 || j.arr[0].kind != Json::Str) fail("malformed dim");
    static const std::map<std::string, Dim::Op> ops = {{"+", Dim::Add},  {"*", Dim::Mul},   {"//", Dim::FloorDiv},
                                                        {"%", Dim::Mod},  {"max", Dim::Max}, {"min", Dim::Min}};
    const auto op = ops.find(j.arr[0].s);
    if (op == ops.end()) fail("unknown dim operator '" + j.arr[0].s + "'");
    Dim d = parse_dim(j.arr[1], syms);
    for (size_t k = 2; k < j.arr.size(); k++) d.fold(op->second, parse_dim(j.arr[k], syms));
    return d;
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
    Dim ne_x[4];
    std::vector<Dim> shape_x;
    int64_t ne[4] = {1, 1, 1, 1};  // for the current binding

    bool symbolic() const {
        for (const auto & d : ne_x)
            if (!d.fixed()) return true;
        return false;
    }
    void bind(const std::vector<int64_t> & b) {
        for (int k = 0; k < 4; k++) {
            ne[k] = ne_x[k](b);
            if (ne[k] < 1) fail("value '" + name + "' gets a dim of " + std::to_string(ne[k]));
        }
    }
    std::vector<int64_t> shape(const std::vector<int64_t> & b) const {
        std::vector<int64_t> s;
        for (const auto & d : shape_x) s.push_back(d(b));
        return s;
    }
    size_t nbytes(const std::vector<int64_t> & b) const {
        return ggml_row_size((ggml_type) type, ne_x[0](b)) * (size_t) (ne_x[1](b) * ne_x[2](b) * ne_x[3](b));
    }
};

void parse_ne(const Json & j, const std::vector<Symbol> & syms, Dim (&ne)[4]) {
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
    Dim ne_x[4];
    int64_t ne[4] = {1, 1, 1, 1};
    Json p;                                        // op parameters
    std::vector<std::pair<std::string, Dim>> p_x;  // symbolic ones (a view's start)
    std::map<std::string, int64_t> p_bound;        // their values for the binding

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
    // loop
    int n = 0, n_symbol = -1;
    std::vector<std::pair<std::string, std::string>> counters, collect, carry, slices;
    std::vector<std::pair<int, Dim>> bind;
    std::vector<std::pair<std::string, int>> masks;
    std::vector<std::pair<std::string, std::vector<int>>> until;
    std::vector<std::pair<std::string, std::vector<float>>> scalars;
    std::vector<DriverOp> body;
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
    // "symbol 'n' = 9 is outside [1, 8]" unless v lies in symbol k's range
    void check_range(int k, int64_t v) const {
        const Symbol & sy = symbols[(size_t) k];
        if (v < sy.min || v > sy.max)
            fail("symbol '" + sy.name + "' = " + std::to_string(v) + " is outside [" + std::to_string(sy.min) + ", " +
                 std::to_string(sy.max) + "]");
    }
    void bind(const std::vector<int64_t> & b) {
        if (b.size() != symbols.size()) fail("binding has the wrong number of symbols");
        for (size_t k = 0; k < symbols.size(); k++) check_range((int) k, b[k]);
        for (auto & v : values) v.bind(b);
        for (auto & s : stages) {
            for (auto & p : s.params) p.bind(b);
            for (auto & n : s.nodes) {
                for (int k = 0; k < 4; k++) n.ne[k] = n.ne_x[k](b);
                for (const auto & kv : n.p_x) n.p_bound[kv.first] = kv.second(b);
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
            for (const auto & d : s.params.back().ne_x) d.mark(used);
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
            for (const auto & d : n.ne_x) d.mark(used);
            for (const char * key : {"start", "stop"})
                if (const Json * v = n.p.find(key); v && v->kind != Json::Num) {
                    n.p_x.emplace_back(key, parse_dim(*v, prog.symbols));
                    n.p_x.back().second.mark(used);
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

// ------------------------------------------------------------------------------- node -> ggml

namespace gcq {
namespace {

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

// The program ops this runtime turns into ggml calls (the op surface of runtime/src/ops.cpp:56-309
// that runs on this library). Shape rules are enforced by the ggml layer, whose constructors refuse
// what ggml would abort on and say why; what the HIP executor cannot run fails supports_op when the
// stage's graph is checked. The loader itself only picks parameters and arities.
enum class NodeOp {
    Add, Sub, Mul, Div, Unary, Mean, SumRows, Clamp, Repeat, Concat, Norm, Cont, MulMat, Scale, RmsNorm, SoftMax,
    Reshape, Permute, View, FlashAttn, Swiglu, SetRows, Rope, Argmax, GetRows, Cast,
};

using UnaryFn = ggml_tensor * (*)(ggml_context *, ggml_tensor *);

struct NodeKind {
    NodeOp op;
    int lo, hi;             // inputs
    UnaryFn fn = nullptr;  // NodeOp::Unary
};

const std::unordered_map<std::string, NodeKind> & node_kinds() {
    static const std::unordered_map<std::string, NodeKind> kinds = [] {
        std::unordered_map<std::string, NodeKind> k = {
            {"add", {NodeOp::Add, 2, 2}},        {"sub", {NodeOp::Sub, 2, 2}},
            {"mul", {NodeOp::Mul, 2, 2}},        {"div", {NodeOp::Div, 2, 2}},
            {"mean", {NodeOp::Mean, 1, 1}},      {"sum_rows", {NodeOp::SumRows, 1, 1}},
            {"clamp", {NodeOp::Clamp, 1, 1}},    {"repeat", {NodeOp::Repeat, 1, 1}},
            {"concat", {NodeOp::Concat, 2, 2}},  {"norm", {NodeOp::Norm, 1, 1}},
            {"cont", {NodeOp::Cont, 1, 1}},      {"mul_mat", {NodeOp::MulMat, 2, 2}},
            {"scale", {NodeOp::Scale, 1, 1}},    {"rms_norm", {NodeOp::RmsNorm, 1, 1}},
            {"soft_max", {NodeOp::SoftMax, 1, 2}}, {"reshape", {NodeOp::Reshape, 1, 1}},
            {"permute", {NodeOp::Permute, 1, 1}}, {"view", {NodeOp::View, 1, 1}},
            {"flash_attn", {NodeOp::FlashAttn, 3, 4}}, {"swiglu", {NodeOp::Swiglu, 2, 2}},
            {"set_rows", {NodeOp::SetRows, 3, 3}}, {"rope", {NodeOp::Rope, 2, 3}},
            {"argmax", {NodeOp::Argmax, 1, 1}},  {"get_rows", {NodeOp::GetRows, 2, 2}},
            {"cast", {NodeOp::Cast, 1, 1}},
        };
        // elementwise functions; gelu_tanh is the tanh form, which is what ggml_gelu computes here
        const std::pair<const char *, UnaryFn> unaries[] = {
            {"relu", ggml_relu}, {"gelu", ggml_gelu},       {"gelu_tanh", ggml_gelu}, {"gelu_erf", ggml_gelu_erf},
            {"silu", ggml_silu}, {"tanh", ggml_tanh},       {"sigmoid", ggml_sigmoid}, {"exp", ggml_exp},
            {"log", ggml_log},   {"neg", ggml_neg},         {"abs", ggml_abs},         {"sqr", ggml_sqr},
            {"sqrt", ggml_sqrt}, {"sin", ggml_sin},         {"cos", ggml_cos},         {"softplus", ggml_softplus},
        };
        for (const auto & u : unaries) k[u.first] = {NodeOp::Unary, 1, 1, u.second};
        return k;
    }();
    return kinds;
}

ggml_tensor * emit_node(ggml_context * ctx, const NodeSpec & n, const std::vector<ggml_tensor *> & s) {
    const auto & kinds = node_kinds();
    const auto it = kinds.find(n.op);
    if (it == kinds.end()) node_fail(n, "op is not supported by this runtime");
    const NodeKind & k = it->second;
    if ((int) s.size() < k.lo || (int) s.size() > k.hi)
        node_fail(n, "expected " + std::to_string(k.lo) + (k.lo == k.hi ? "" : "-" + std::to_string(k.hi)) +
                         " inputs, got " + std::to_string(s.size()));
    auto f = [&](const char * key) { return (float) n.num(key); };
    ggml_tensor * t = nullptr;
    switch (k.op) {
        case NodeOp::Add: t = ggml_add(ctx, s[0], s[1]); break;
        case NodeOp::Sub: t = ggml_sub(ctx, s[0], s[1]); break;
        case NodeOp::Mul: t = ggml_mul(ctx, s[0], s[1]); break;
        case NodeOp::Div: t = ggml_div(ctx, s[0], s[1]); break;
        case NodeOp::Unary: t = k.fn(ctx, s[0]); break;
        case NodeOp::Mean: t = ggml_mean(ctx, s[0]); break;
        case NodeOp::SumRows: t = ggml_sum_rows(ctx, s[0]); break;
        case NodeOp::Clamp: t = ggml_clamp(ctx, s[0], f("min"), f("max")); break;
        case NodeOp::Repeat: t = ggml_repeat_4d(ctx, s[0], n.ne[0], n.ne[1], n.ne[2], n.ne[3]); break;
        case NodeOp::Concat: t = ggml_concat(ctx, s[0], s[1], (int) n.integer("dim")); break;
        case NodeOp::Norm: t = ggml_norm(ctx, s[0], f("eps")); break;
        case NodeOp::Cont: t = ggml_cont(ctx, s[0]); break;
        case NodeOp::MulMat:
            t = ggml_mul_mat(ctx, s[0], s[1]);
            if (t && n.has("acc") && n.integer("acc") != 0) ggml_prec_set_acc(t, GGML_PREC_F32);
            break;
        case NodeOp::Scale: {
            const float b = (float) n.num_or("b", 0.0);
            t = b == 0.0f ? ggml_scale(ctx, s[0], f("s")) : ggml_scale_bias(ctx, s[0], f("s"), b);
            break;
        }
        case NodeOp::RmsNorm: t = ggml_rms_norm(ctx, s[0], f("eps")); break;
        case NodeOp::SoftMax:
            t = ggml_soft_max_ext(ctx, s[0], s.size() > 1 ? s[1] : nullptr, (float) n.num_or("scale", 1.0),
                                  (float) n.num_or("max_bias", 0.0));
            break;
        case NodeOp::Reshape:
            if (ggml_nelements(s[0]) != n.ne[0] * n.ne[1] * n.ne[2] * n.ne[3])
                node_fail(n, "cannot reshape " + ne_str(s[0]->ne) + " to " + ne_str(n.ne));
            t = reshape_of(ctx, s[0], n.ne);
            if (!t)
                node_fail(n, "input is a strided view and the reshape does more than add or drop size-1 dims; it "
                             "needs a cont first");
            break;
        case NodeOp::Permute: {
            const Json * ax = n.p.find("axes");
            if (!ax || ax->items().size() != 4) node_fail(n, "'axes' must have 4 entries");
            t = ggml_permute(ctx, s[0], (int) ax->arr[0].as_int(), (int) ax->arr[1].as_int(),
                             (int) ax->arr[2].as_int(), (int) ax->arr[3].as_int());
            break;
        }
        case NodeOp::View: {
            const int64_t dim = n.integer("dim"), start = n.integer("start");
            if (dim < 0 || dim > 3 || start < 0 || start + n.ne[dim] > s[0]->ne[dim])
                node_fail(n, "slice out of range of " + ne_str(s[0]->ne));
            t = slice_of(ctx, s[0], (int) dim, start, n.ne);
            break;
        }
        case NodeOp::FlashAttn:
            t = ggml_flash_attn_ext(ctx, s[0], s[1], s[2], s.size() > 3 ? s[3] : nullptr, f("scale"), 0.0f, 0.0f);
            if (t) ggml_prec_set_acc(t, GGML_PREC_F32);
            break;
        case NodeOp::Swiglu: t = ggml_swiglu_split(ctx, s[0], s[1]); break;
        case NodeOp::SetRows: t = ggml_set_rows(ctx, s[0], s[1], s[2]); break;
        case NodeOp::Rope:
            t = ggml_rope_ext(ctx, s[0], s[1], s.size() > 2 ? s[2] : nullptr, (int) n.integer("n_dims"),
                              (int) n.integer("mode"), 0, f("freq_base"), f("freq_scale"), 0.0f, f("attn_factor"),
                              32.0f, 1.0f);
            break;
        case NodeOp::Argmax: t = ggml_argmax(ctx, s[0]); break;
        case NodeOp::GetRows: t = ggml_get_rows(ctx, s[0], s[1]); break;
        case NodeOp::Cast: t = ggml_cast(ctx, s[0], (ggml_type) n.type); break;
    }
    if (!t) node_fail(n, std::string("ggml could not build it: ") + ggml_last_error());
    if (t->type != n.type)
        node_fail(n, std::string("produced type ") + ggml_type_name(t->type) + ", program expects " +
                         ggml_type_name((ggml_type) n.type));
    for (int q = 0; q < 4; q++)
        if (t->ne[q] != n.ne[q]) node_fail(n, "produced shape " + ne_str(t->ne) + ", program expects " + ne_str(n.ne));
    ggml_set_name(t, n.id.c_str());
    return t;
}

}  // namespace
}  // namespace gcq

// ------------------------------------------------------------------------ device-side driver work

namespace gcq {
namespace {

// The small work a driver does between its graphs (scalar and counter fills, causal mask rows,
// slice and collect copies), several of them in one launch: op blockIdx.y, element i.
enum { D_FILL32, D_CAUSAL, D_COPY4, D_COPY1, D_COPY4_IF, D_COPY1_IF, D_UNTIL };
constexpr int kDriverBatch = 8;
constexpr size_t kDriverCopyMax = 1 << 20;  // larger copies: hipMemcpyAsync
struct DriverKOp {
    int kind;
    uint32_t bits;
    int64_t n, len, pos;  // elements; D_CAUSAL: row length and position; _IF / D_UNTIL: the iteration
    uint8_t * dst;
    const uint8_t * src;
    const int32_t * aux;  // _IF: the loop's stop word; D_UNTIL: its len stop ids
    int32_t * host;       // D_UNTIL: host-visible {stop, iterations done}
    // Iteration-relative forms (a loop iteration captured once and replayed): with `it` (the
    // loop's iteration word on the device) set, the op is for iteration it = *it: dst and src
    // advance by dstep / sstep bytes per iteration (ring: dst alternates between two slots,
    // dstep apart), a position or D_FILL32 value adds it to the word at `base` (a counter's
    // start), a D_FILL32 value comes from the table `tab` at it, and _IF / D_UNTIL take pos = it.
    const int32_t * it;
    const int32_t * base;
    const uint32_t * tab;
    int64_t dstep, sstep;
    int ring;
};
struct DriverBatch {
    DriverKOp op[kDriverBatch];
    int32_t * advance;  // a launch of one workgroup: this iteration word steps once every op has read it
};

__device__ __forceinline__ void driver_op(const DriverKOp & o, int64_t i) {
    if (i >= o.n) return;
    const int64_t it = o.it ? (int64_t) *o.it : 0;
    uint8_t * dst = o.dst + (o.ring ? (it & 1) : it) * o.dstep;
    const uint8_t * src = o.src ? o.src + it * o.sstep : nullptr;
    const int64_t base = o.base ? (int64_t) *o.base + it : 0;  // a counter's value at iteration it
    const int64_t pos = o.it ? (o.base ? base : it) : o.pos;
    switch (o.kind) {
        case D_FILL32:
            reinterpret_cast<uint32_t *>(dst)[i] = o.tab ? o.tab[it] : o.base ? (uint32_t) base : o.bits;
            break;
        // rows of a causal mask for position pos: 0 where the key index (element % len) is <= pos
        case D_CAUSAL: reinterpret_cast<float *>(dst)[i] = i % o.len <= pos ? 0.0f : -INFINITY; break;
        case D_COPY4: reinterpret_cast<uint32_t *>(dst)[i] = reinterpret_cast<const uint32_t *>(src)[i]; break;
        // a collected row of an iteration at or before the loop's stop (the stop word holds the
        // iteration whose value met the until ids, or INT32_MAX)
        case D_COPY4_IF:
            if (pos <= *o.aux) reinterpret_cast<uint32_t *>(dst)[i] = reinterpret_cast<const uint32_t *>(src)[i];
            break;
        case D_COPY1_IF:
            if (pos <= *o.aux) dst[i] = src[i];
            break;
        // the until test of iteration pos: the stop word takes pos if the value is one of the ids;
        // then the host's copy of the stop word, then the iterations done (its release)
        case D_UNTIL: {
            const int32_t v = *reinterpret_cast<const int32_t *>(src);
            bool hit = false;
            for (int64_t k = 0; k < o.len; k++) hit = hit || o.aux[k] == v;
            int32_t * stop = reinterpret_cast<int32_t *>(dst);
            int32_t cur = *stop;
            if (hit && cur > (int32_t) pos) {
                cur = (int32_t) pos;
                *stop = cur;
            }
            __hip_atomic_store(&o.host[0], cur, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __hip_atomic_store(&o.host[1], (int32_t) (pos + 1), __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
            break;
        }
        default: dst[i] = src[i]; break;
    }
}

__global__ void k_driver_ops(const DriverBatch b) {
    driver_op(b.op[blockIdx.y], (int64_t) blockIdx.x * blockDim.x + threadIdx.x);
    if (b.advance) {  // the launch is one workgroup: every read of the word is before the barrier
        __syncthreads();
        if (threadIdx.x == 0) *b.advance += 1;
    }
}

// The last launch of a captured loop iteration when its ops take several workgroups: the loop's
// iteration word moves to the next.
__global__ void k_iter_next(int32_t * it) {
    if (threadIdx.x == 0) *it += 1;
}

// The work a driver does between its graphs, ordered on the backend's stream with them, so a loop
// iteration waits for the host only where the host must see a value (a counter's start, an until
// token). Fills, mask rows and small copies wait in a batch that one launch runs before the next
// graph, copy, read or wait (a loop iteration's counter, mask and the previous iteration's
// collected row: one launch); an op touching memory a waiting one writes, or writing memory one
// reads, runs the batch first, so the ops keep their order's effect.
class StreamOps {
  public:
    void attach(ggml_backend_t be) {
        s_ = backend_stream(be);
        check_hip(hipHostMalloc(&pinned_, 64, hipHostMallocDefault), "hipHostMalloc");
    }
    ~StreamOps() {
        if (pinned_) (void) hipHostFree(pinned_);
    }
    void fill32(void * p, int64_t n, uint32_t bits) {
        if (n <= 0) return;
        add({D_FILL32, bits, n, 0, 0, (uint8_t *) p, nullptr, nullptr, nullptr}, (size_t) n * 4);
    }
    void causal(float * p, int64_t n, int64_t len, int64_t pos) {
        if (n <= 0) return;
        add({D_CAUSAL, 0, n, len, pos, (uint8_t *) p, nullptr, nullptr, nullptr}, (size_t) n * 4);
    }
    void copy(void * dst, const void * src, size_t n) {
        if (!n) return;
        if (n > kDriverCopyMax) {
            flush();
            check_hip(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, s_), "driver copy");
            return;
        }
        const bool words = ((uintptr_t) dst & 3) == 0 && ((uintptr_t) src & 3) == 0 && n % 4 == 0;
        add({words ? D_COPY4 : D_COPY1, 0, (int64_t) (words ? n / 4 : n), 0, 0, (uint8_t *) dst,
             (const uint8_t *) src, nullptr, nullptr},
            n);
    }
    // copy if iteration `it` is at or before the stop word's iteration
    void copy_if(void * dst, const void * src, size_t n, const int32_t * stop, int64_t it) {
        if (!n) return;
        const bool words = ((uintptr_t) dst & 3) == 0 && ((uintptr_t) src & 3) == 0 && n % 4 == 0;
        DriverKOp o{words ? D_COPY4_IF : D_COPY1_IF, 0, (int64_t) (words ? n / 4 : n), 0, it, (uint8_t *) dst,
                    (const uint8_t *) src, stop, nullptr};
        add(o, n);
    }
    void until(const int32_t * value, const int32_t * ids, int64_t n_ids, int32_t * stop, int32_t * host, int64_t it) {
        DriverKOp o{D_UNTIL, 0, 1, n_ids, it, (uint8_t *) stop, (const uint8_t *) value, ids, host};
        add(o, 4);
    }
    // Iteration-relative ops (DriverKOp::it): for a loop iteration captured once and replayed.
    // span: the bytes an op may touch over all iterations (from dst / src), for the batch's
    // overlap check.
    void fill32_tab(void * p, int64_t n, const uint32_t * tab, const int32_t * it) {
        DriverKOp o{D_FILL32, 0, n, 0, 0, (uint8_t *) p, nullptr, nullptr, nullptr};
        o.it = it, o.tab = tab;
        add(o, (size_t) n * 4);
    }
    void fill32_ctr(void * p, int64_t n, const int32_t * base, const int32_t * it) {
        DriverKOp o{D_FILL32, 0, n, 0, 0, (uint8_t *) p, nullptr, nullptr, nullptr};
        o.it = it, o.base = base;
        add(o, (size_t) n * 4);
    }
    void causal_rel(float * p, int64_t n, int64_t len, const int32_t * base, const int32_t * it) {
        DriverKOp o{D_CAUSAL, 0, n, len, 0, (uint8_t *) p, nullptr, nullptr, nullptr};
        o.it = it, o.base = base;
        add(o, (size_t) n * 4);
    }
    // dst + step(it) <- src + it * sstep, n bytes (at most kDriverCopyMax); step(it) = it * dstep,
    // or (it & 1) * dstep for a ring
    void copy_rel(void * dst, const void * src, size_t n, int64_t dstep, int64_t sstep, bool ring, const int32_t * it,
                  size_t dspan, size_t sspan) {
        require(n <= kDriverCopyMax, "driver: iteration copy too large");
        const bool words = ((uintptr_t) dst & 3) == 0 && ((uintptr_t) src & 3) == 0 && n % 4 == 0 && dstep % 4 == 0 &&
                           sstep % 4 == 0;
        DriverKOp o{words ? D_COPY4 : D_COPY1, 0, (int64_t) (words ? n / 4 : n), 0, 0, (uint8_t *) dst,
                    (const uint8_t *) src, nullptr, nullptr};
        o.it = it, o.dstep = dstep, o.sstep = sstep, o.ring = ring;
        add(o, dspan, sspan);
    }
    void copy_if_rel(void * dst, const void * src, size_t n, int64_t dstep, const int32_t * stop, const int32_t * it,
                     size_t dspan) {
        require(n <= kDriverCopyMax, "driver: iteration copy too large");
        const bool words = ((uintptr_t) dst & 3) == 0 && ((uintptr_t) src & 3) == 0 && n % 4 == 0 && dstep % 4 == 0;
        DriverKOp o{words ? D_COPY4_IF : D_COPY1_IF, 0, (int64_t) (words ? n / 4 : n), 0, 0, (uint8_t *) dst,
                    (const uint8_t *) src, stop, nullptr};
        o.it = it, o.dstep = dstep;
        add(o, dspan, n);
    }
    void until_rel(const int32_t * value, const int32_t * ids, int64_t n_ids, int32_t * stop, int32_t * host,
                   const int32_t * it) {
        DriverKOp o{D_UNTIL, 0, 1, n_ids, 0, (uint8_t *) stop, (const uint8_t *) value, ids, host};
        o.it = it;
        add(o, 4);
    }
    // the waiting ops, then the loop's iteration word to the next iteration: in the same launch
    // when the ops take one workgroup, else a launch of its own
    void iter_next(int32_t * it) {
        int64_t most = 0;
        for (int k = 0; k < n_; k++) most = std::max(most, b_.op[k].n);
        if (n_ == 1 && most <= 256) {
            b_.advance = it;
            flush();
            return;
        }
        flush();
        k_iter_next<<<1, 64, 0, s_>>>(it);
        check_launch("driver iteration");
    }
    void clear(void * dst, size_t n) {
        flush();
        if (n) check_hip(hipMemsetAsync(dst, 0, n, s_), "driver clear");
    }
    int32_t read_i32(const void * src) {
        flush();
        check_hip(hipMemcpyAsync(pinned_, src, 4, hipMemcpyDeviceToHost, s_), "driver read");
        check_hip(hipStreamSynchronize(s_), "driver read");
        int32_t v;
        std::memcpy(&v, pinned_, 4);
        return v;
    }
    void finish() {
        flush();
        check_hip(hipStreamSynchronize(s_), "driver");
    }
    // the stream, with every waiting op launched on it
    hipStream_t stream() {
        flush();
        return s_;
    }
    // ops left waiting by a run that failed: never launched
    void discard() {
        n_ = 0;
        b_.advance = nullptr;
    }
    void flush() {
        if (n_ == 0) return;
        int64_t most = 0;
        for (int k = 0; k < n_; k++) most = std::max(most, b_.op[k].n);
        k_driver_ops<<<dim3((unsigned) ((most + 255) / 256), (unsigned) n_), 256, 0, s_>>>(b_);
        n_ = 0;
        b_.advance = nullptr;
        check_launch("driver ops");
    }

  private:
    void add(const DriverKOp & o, size_t bytes) { add(o, bytes, bytes); }
    void add(const DriverKOp & o, size_t wbytes, size_t rbytes) {
        const uintptr_t w0 = (uintptr_t) o.dst, w1 = w0 + wbytes;
        const uintptr_t r0 = (uintptr_t) o.src, r1 = o.src ? r0 + rbytes : r0;
        bool clash = n_ == kDriverBatch;
        for (int k = 0; k < n_ && !clash; k++) {
            const uintptr_t pw0 = wr_[k][0], pw1 = wr_[k][1], pr0 = rd_[k][0], pr1 = rd_[k][1];
            clash = (w0 < pw1 && pw0 < w1) || (r0 < pw1 && pw0 < r1) || (w0 < pr1 && pr0 < w1);
        }
        if (clash) flush();
        wr_[n_][0] = w0;
        wr_[n_][1] = w1;
        rd_[n_][0] = r0;
        rd_[n_][1] = r1;
        b_.op[n_++] = o;
    }
    hipStream_t s_ = nullptr;
    void * pinned_ = nullptr;
    DriverBatch b_{};
    int n_ = 0;
    uintptr_t wr_[kDriverBatch][2], rd_[kDriverBatch][2];  // byte ranges each waiting op writes / reads
};

// GPU time per stage: one event after each call (and one before a run's first), read after the
// run's final wait. A call's time runs from the event before it (the previous call's, or the
// run's first) to its own, so driver work between two calls counts with the call after it; one
// event per call instead of a pair, and events without a system-scope release (the host reads
// results only after the stream's final wait), since every event costs the stream a few us. A
// loop iteration replayed from its captured graph has one event for all of its calls; its time is
// split over the body's stages as the same loop's uncaptured iterations of the run split theirs.
class StageClock {
  public:
    ~StageClock() {
        for (hipEvent_t e : events_) (void) hipEventDestroy(e);
    }
    void begin_run() {
        marks_.clear();
        used_ = 0;
    }
    // before a call: the run's first event, if this is its first call
    void before(hipStream_t s) {
        if (used_ == 0) record(s);
    }
    // after a call of stage `stage`; group: the loop (with captured iterations) it belongs to, or -1
    void after(int stage, hipStream_t s, int group = -1) {
        marks_.push_back({stage, used_ - 1, used_, group, nullptr, false});
        record(s);
    }
    // after a captured iteration of loop `group`, whose body calls the stages in `body`
    void after_iteration(int group, const std::vector<int> * body, hipStream_t s) {
        marks_.push_back({-1, used_ - 1, used_, group, body, false});
        record(s);
    }
    size_t marks() const { return marks_.size(); }
    // calls from mark k on are not counted (a loop iteration that ran past the loop's end)
    void forget_since(size_t k) {
        for (size_t i = k; i < marks_.size(); i++) marks_[i].dead = true;
    }
    // ms and calls of each stage, accumulated into per-stage totals: add(stage, ms, calls)
    template <class F>
    void collect(F && add) {
        std::map<int, std::map<int, double>> share;  // loop -> stage -> ms of its uncaptured calls
        std::vector<float> ms(marks_.size(), 0.0f);
        for (size_t k = 0; k < marks_.size(); k++) {
            const Mark & m = marks_[k];
            if (m.dead) continue;
            check_hip(hipEventElapsedTime(&ms[k], events_[m.start], events_[m.stop]), "hipEventElapsedTime");
            if (m.body) continue;
            add(m.stage, (double) ms[k], 1);
            if (m.group >= 0) share[m.group][m.stage] += ms[k];
        }
        for (size_t k = 0; k < marks_.size(); k++) {
            const Mark & m = marks_[k];
            if (m.dead || !m.body || m.body->empty()) continue;
            std::map<int, int> calls;
            for (int st : *m.body) calls[st]++;
            double total = 0.0;
            for (const auto & c : calls) total += share[m.group][c.first];
            for (const auto & c : calls) {
                const double part = total > 0.0 ? share[m.group][c.first] / total
                                                : (double) c.second / (double) m.body->size();
                add(c.first, (double) ms[k] * part, c.second);
            }
        }
    }

  private:
    void record(hipStream_t s) {
        if (used_ == events_.size()) {
            hipEvent_t e;
            check_hip(hipEventCreateWithFlags(&e, hipEventDisableSystemFence), "hipEventCreate");
            events_.push_back(e);
        }
        check_hip(hipEventRecord(events_[used_], s), "hipEventRecord");
        used_++;
    }
    struct Mark {
        int stage;
        size_t start, stop;
        int group;
        const std::vector<int> * body;  // a captured iteration's stages, else nullptr
        bool dead;
    };
    std::vector<hipEvent_t> events_;
    std::vector<Mark> marks_;
    size_t used_ = 0;
};

// GGML_COMPILER_LOG=debug: the runtime's informational messages on stderr (warnings always).
bool log_debug() {
    static const bool on = [] {
        const char * e = std::getenv("GGML_COMPILER_LOG");
        return e && std::strcmp(e, "debug") == 0;
    }();
    return on;
}

// Runs f, which calls the ggml API's void functions (errors recorded, not thrown); throws with
// `what` if any of them recorded one.
template <class F>
void ggml_checked(const std::string & what, F && f) {
    const uint64_t before = error_count();
    f();
    if (error_count() != before) fail(what + ": " + last_error());
}

}  // namespace
}  // namespace gcq

// ------------------------------------------------------------------------------------ model

using namespace gcq;

struct ggml_compiler_stage_build {
    ggml_context * ctx = nullptr;
    ggml_backend_t backend = nullptr;
    ggml_context * wctx = nullptr;
    const std::vector<int64_t> * binding = nullptr;
    std::vector<ggml_tensor *> params, outputs;
    std::string error;
};

namespace gcq {
namespace {

// One driver call of a stage: the stage's graph built over the driver values it reads and writes.
struct CallGraph {
    int stage = -1;
    const DriverOp * op = nullptr;
    // the graph in use: of the current binding, for a stage whose shapes read a symbol
    ggml_context * ctx = nullptr;
    ggml_cgraph * graph = nullptr;
    ggml_gallocr_t alloc = nullptr;
    bool stale = false;  // no graph for the current binding yet: built before its next run
    // A symbolic stage's graphs per binding (the model keeps a few bindings' views), each with its
    // own allocation, so a binding seen again reuses its graph and the executor's capture of it.
    struct Build {
        std::vector<int64_t> binding;
        ggml_context * ctx = nullptr;
        ggml_cgraph * graph = nullptr;
        ggml_gallocr_t alloc = nullptr;
    };
    std::vector<Build> builds;

    void drop_graph() {
        if (ctx) ggml_free(ctx);
        ctx = nullptr;
        graph = nullptr;
    }
    void use(const Build & b) {
        ctx = b.ctx;
        graph = b.graph;
        alloc = b.alloc;
        stale = false;
    }
    void forget(const std::vector<int64_t> & binding) {
        for (size_t k = 0; k < builds.size();) {
            if (builds[k].binding != binding) {
                k++;
                continue;
            }
            if (builds[k].graph == graph) ctx = nullptr, graph = nullptr, alloc = nullptr, stale = true;
            if (builds[k].ctx) ggml_free(builds[k].ctx);
            if (builds[k].alloc) ggml_gallocr_free(builds[k].alloc);
            builds.erase(builds.begin() + (long) k);
        }
    }
    void free_all() {
        for (Build & b : builds) {
            if (b.ctx) ggml_free(b.ctx);
            if (b.alloc) ggml_gallocr_free(b.alloc);
        }
        if (builds.empty()) {  // a stage without symbols: its one graph
            if (alloc) ggml_gallocr_free(alloc);
            drop_graph();
        }
        builds.clear();
        ctx = nullptr, graph = nullptr, alloc = nullptr;
    }
};

// A driver compiled to flat code: calls, and loops as enter / top / bottom with jumps.
struct VmCode {
    enum Kind : uint8_t { Call, Enter, Top, Bottom };
    Kind kind;
    const DriverOp * op;
    int jump;  // Top: the instruction after its Bottom; Bottom: its Top
    int call;  // Call: index into the model's call graphs
};

// A loop's until test on the device (one int32 until value): its stop word and ids, the values
// its body writes (state aside) as of the last two iterations, and a host-visible {stop,
// iterations done} that the iterations' test ops write.
//
// Such a loop's iterations can also be captured once into a HIP graph and replayed: every op of
// an iteration then has an iteration-relative form (DriverKOp::it) reading the loop's iteration
// word `it` on the device, the counters' starts from `base` and the scalars from device tables,
// and the last launch of the iteration moves `it` on. One graph per binding of the symbols (and
// executor workspace epoch); the stages' graphs run inside it as plain launches.
constexpr int kUntilCounters = 16;  // counters a captured loop may have
struct UntilState {
    void * dev = nullptr;          // [stop word, iteration word, counter starts] [ids] [per kept value: two slots]
    int32_t * stop = nullptr;
    int32_t * it = nullptr;
    int32_t * base = nullptr;      // kUntilCounters words
    int32_t * ids = nullptr;
    int64_t n_ids = 0;
    std::vector<std::string> kept;  // the values the body writes, state aside
    std::vector<uint8_t *> ring;    // per kept value: slot (iteration & 1)
    std::vector<size_t> slot_bytes;
    int32_t * host = nullptr;      // pinned
    // captured iterations
    bool has_until = false;        // the until test runs on the device (else the loop has none)
    int group = -1;                // the loop's tag in the stage clock
    bool graphable = false;        // every op of an iteration has an iteration-relative form
    void * tab_mem = nullptr;      // the scalars' per-iteration values
    std::vector<const uint32_t *> tabs;
    std::vector<int> body_stages;  // the stage of each body call, in order
    struct IterGraph {
        std::vector<int64_t> binding;
        uint64_t epoch;
        hipGraphExec_t exec;
    };
    std::vector<IterGraph> graphs;
    void drop_graphs(const std::vector<int64_t> * binding) {
        for (size_t k = 0; k < graphs.size();) {
            if (binding && graphs[k].binding != *binding) {
                k++;
                continue;
            }
            (void) hipGraphExecDestroy(graphs[k].exec);
            graphs.erase(graphs.begin() + (long) k);
        }
    }
    UntilState() = default;
    UntilState(const UntilState &) = delete;
    UntilState & operator=(const UntilState &) = delete;
    ~UntilState() {
        drop_graphs(nullptr);
        if (dev) (void) hipFree(dev);
        if (tab_mem) (void) hipFree(tab_mem);
        if (host) (void) hipHostFree(host);
    }
};

struct LoopFrame {
    const DriverOp * op;
    int trips, i;
    std::vector<int32_t> start;  // counters' values at loop entry
    UntilState * until = nullptr;  // the until test on the device, when the loop has one
    UntilState * cap = nullptr;    // the loop's device state for captured iterations (a body of calls)
    uint64_t calls0 = 0;           // calls made and stage-clock marks before this iteration
    size_t marks0 = 0;
    bool replayed = false;         // this iteration ran as its loop's captured graph
};

}  // namespace
}  // namespace gcq

struct ggml_compiler_model {
    // ---- what was loaded
    Program prog;
    GgufFile file;
    std::map<std::string, ggml_compiler_build_fn> builders;
    ggml_backend_t backend = nullptr;
    ggml_context * wctx = nullptr;  // weights and constants, one HIP buffer
    ggml_backend_buffer_t wbuf = nullptr;
    // ---- driver values: storage sized for the largest binding, views for the current one
    ggml_context * vctx = nullptr;
    ggml_backend_buffer_t vbuf = nullptr;
    // Driver values of symbolic shape viewed per binding, the last kKeepBindings bindings used.
    static constexpr size_t kKeepBindings = 8;
    struct ViewSet {
        std::vector<int64_t> binding;
        ggml_context * ctx = nullptr;
        std::unordered_map<std::string, ggml_tensor *> views;
        uint64_t used = 0;
    };
    std::vector<ViewSet> view_sets;
    uint64_t view_clock = 0;
    std::unordered_map<std::string, const TensorSpec *> spec;
    std::unordered_map<std::string, ggml_tensor *> storage, bound;
    std::set<std::string> inputs_set;  // inputs given since load
    // ---- symbols: the binding the next run uses, the one the views and graphs were made for
    std::vector<int64_t> binding, built;
    // ---- compiled drivers and their call graphs
    struct Entry {
        const EntrySpec * spec = nullptr;
        std::vector<const TensorSpec *> in, out;
        std::vector<VmCode> code;
    };
    std::vector<Entry> entries;
    std::vector<CallGraph> calls;
    // ---- running
    std::map<const DriverOp *, std::unique_ptr<UntilState>> untils;
    int cur_group = -1;  // the stage-clock tag of the loop whose body is running, or -1
    StreamOps ops;
    StageClock clock;
    std::vector<ggml_compiler_stats> stage_totals;  // ms_total, n_calls per stage
    ggml_compiler_stats last{};
    struct ProfileLine {
        std::string stage, node, op;
        double ms;
    };
    std::vector<ProfileLine> profile;
    // GGML_COMPILER_PROFILE=<file>, read when the model loads: every graph runs one node at a time,
    // waited for, and after each run "stage<TAB>node<TAB>op<TAB>ms" lines are appended to <file>
    // (the reference runtime's profile, runtime/src/ggml_compiler_rt.cpp:83-88, 219-240, 343-354,
    // which reads the variable once per process). Fusion is off in this mode, so every node is one
    // launch of its own.
    std::string profile_path;
    const char * profile_file() const { return profile_path.empty() ? nullptr : profile_path.c_str(); }

    ~ggml_compiler_model() {
        if (backend) (void) hipStreamSynchronize(backend_stream(backend));
        for (auto & c : calls) c.free_all();
        for (auto & v : view_sets)
            if (v.ctx) ggml_free(v.ctx);
        if (vbuf) ggml_backend_buffer_free(vbuf);
        if (vctx) ggml_free(vctx);
        if (wbuf) ggml_backend_buffer_free(wbuf);
        if (wctx) ggml_free(wctx);
        if (backend) ggml_backend_free(backend);
    }

    // ------------------------------------------------------------------------------ loading

    void open(const char * path, const ggml_compiler_options & o) {
        if (o.allow_cpu_fallback) fail("allow_cpu_fallback is not available: this runtime runs on HIP devices only");
        if (o.backend != GGML_COMPILER_BACKEND_HIP && o.backend != GGML_COMPILER_BACKEND_AUTO)
            fail("backend " + std::to_string((int) o.backend) + " is not available: this runtime has the HIP backend "
                 "(GGML_COMPILER_BACKEND_HIP or _AUTO)");
        if (const char * e = std::getenv("GGML_COMPILER_PROFILE")) profile_path = e;
        file.open(path);
        const auto text = file.strings.find("ggml_compiler.program");
        if (text == file.strings.end())
            fail(std::string("'") + path + "' has no ggml_compiler.program; it was not written by ggml-compiler compile");
        prog = parse_program(text->second);
        const int devices = gcq_device_count();
        if (devices == 0) fail("no HIP device");
        if (o.device < 0 || o.device >= devices)
            fail("device index " + std::to_string(o.device) + " out of range; " + std::to_string(devices) +
                 " HIP device(s) found");
        backend = ggml_backend_hip_init(o.device);
        if (!backend) fail(std::string("cannot start the HIP backend: ") + last_error());
        if (profile_file()) {  // nodes one by one: unfused, and no graph capture of single nodes
            backend_set_fusion(backend, false);
            ggml_backend_hip_set_use_graphs(backend, false);
        }
        ops.attach(backend);
        if (log_debug())
            std::fprintf(stderr, "ggml_compiler: %s on %s, %zu tensors, %zu stages, %zu entries\n", path,
                         ggml_backend_name(backend), file.tensors.size(), prog.stages.size(), prog.entries.size());
        upload_tensors();
        for (const auto & sy : prog.symbols) binding.push_back(sy.max);
        prog.bind(binding);
        create_values();
        link_entries();
        stage_totals.assign(prog.stages.size(), ggml_compiler_stats{});
        make_views();
        for (auto & e : entries) compile(e);
        built = binding;
    }

    void upload_tensors() {
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
            for (size_t got = 0; got < n;) {
                const ssize_t r = ::pread(fd, staging.data() + got, n - got, (off_t) (file.data_offset + in.offset + got));
                if (r <= 0) fail("short read for tensor " + in.name);
                got += (size_t) r;
            }
            ggml_checked("upload of tensor " + in.name, [&] { ggml_backend_tensor_set(t, staging.data(), 0, n); });
        }
    }

    // Largest element count of a value over its symbols' ranges. Dims grow with each symbol, so
    // one of the corners of the box of ranges holds it.
    int64_t largest_count(const TensorSpec & v) const {
        std::vector<bool> used(prog.symbols.size(), false);
        for (const auto & d : v.ne_x) d.mark(used);
        std::vector<size_t> free_syms;
        for (size_t k = 0; k < used.size(); k++)
            if (used[k]) free_syms.push_back(k);
        if (free_syms.size() > 20) fail("value '" + v.name + "' depends on too many symbols");
        std::vector<int64_t> b = binding;
        int64_t best = 0;
        for (uint32_t corner = 0; corner < (1u << free_syms.size()); corner++) {
            for (size_t q = 0; q < free_syms.size(); q++) {
                const Symbol & sy = prog.symbols[free_syms[q]];
                b[free_syms[q]] = (corner >> q) & 1u ? sy.max : sy.min;
            }
            int64_t count = 1;
            for (const auto & d : v.ne_x) count *= d(b);
            best = std::max(best, count);
        }
        return best;
    }

    void create_values() {
        ggml_init_params ip{};
        ip.mem_size = ggml_tensor_overhead() * (prog.values.size() + 1);
        ip.no_alloc = true;
        vctx = ggml_init(ip);
        for (const auto & v : prog.values) {
            ggml_tensor * t = v.symbolic() ? ggml_new_tensor_1d(vctx, (ggml_type) v.type, largest_count(v))
                                           : ggml_new_tensor_4d(vctx, (ggml_type) v.type, v.ne[0], v.ne[1], v.ne[2], v.ne[3]);
            if (!t) fail("driver value '" + v.name + "': " + last_error());
            ggml_set_name(t, v.name.c_str());
            storage[v.name] = bound[v.name] = t;
            spec[v.name] = &v;
        }
        if (prog.values.empty()) return;
        vbuf = ggml_backend_alloc_ctx_tensors(vctx, backend);
        if (!vbuf) fail(std::string("cannot allocate driver value buffer: ") + last_error());
        ggml_checked("clearing the driver values", [&] { ggml_backend_buffer_clear(vbuf, 0); });  // state starts at 0
    }

    const TensorSpec & declared(const std::string & name, const char * role) const {
        const auto it = spec.find(name);
        if (it == spec.end()) fail(std::string(role) + " '" + name + "' is not a declared value");
        return *it->second;
    }

    void link_entries() {
        for (const auto & e : prog.entries) {
            Entry en;
            en.spec = &e;
            for (const auto & name : e.inputs) en.in.push_back(&declared(name, "input"));
            for (const auto & name : e.outputs) en.out.push_back(&declared(name, "output"));
            entries.push_back(std::move(en));
        }
        for (const auto & name : prog.state) (void) declared(name, "state");
    }

    // The current binding's view of every symbolic value (same storage, the binding's shape).
    // The driver values of symbolic shape, viewed at the current binding: a binding among the
    // last kKeepBindings reuses its views (which its stages' graphs read); past that the least
    // recently used binding's views and graphs are dropped.
    void make_views() {
        size_t n = 0;
        for (const auto & v : prog.values) n += v.symbolic();
        if (n == 0) return;
        for (ViewSet & vs : view_sets)
            if (vs.binding == binding) {
                vs.used = ++view_clock;
                for (const auto & kv : vs.views) bound[kv.first] = kv.second;
                return;
            }
        if (view_sets.size() >= kKeepBindings) {
            size_t old = 0;
            for (size_t k = 1; k < view_sets.size(); k++)
                if (view_sets[k].used < view_sets[old].used) old = k;
            for (auto & c : calls) c.forget(view_sets[old].binding);
            for (auto & u : untils) u.second->drop_graphs(&view_sets[old].binding);
            ggml_free(view_sets[old].ctx);
            view_sets.erase(view_sets.begin() + (long) old);
        }
        ViewSet vs;
        vs.binding = binding;
        vs.used = ++view_clock;
        ggml_init_params ip{};
        ip.mem_size = ggml_tensor_overhead() * (n + 1);
        ip.no_alloc = true;
        vs.ctx = ggml_init(ip);
        for (const auto & v : prog.values) {
            if (!v.symbolic()) continue;
            const size_t nb1 = ggml_row_size((ggml_type) v.type, v.ne[0]), nb2 = nb1 * (size_t) v.ne[1];
            ggml_tensor * t = ggml_view_4d(vs.ctx, storage.at(v.name), v.ne[0], v.ne[1], v.ne[2], v.ne[3], nb1, nb2,
                                           nb2 * (size_t) v.ne[2], 0);
            if (!t || ggml_backend_view_init(t) != GGML_STATUS_SUCCESS) {
                ggml_free(vs.ctx);
                fail("cannot view driver value '" + v.name + "'");
            }
            ggml_set_name(t, v.name.c_str());
            vs.views[v.name] = t;
            bound[v.name] = t;
        }
        view_sets.push_back(std::move(vs));
    }

    ggml_tensor * value(const std::string & name) const {
        const auto it = bound.find(name);
        if (it == bound.end()) fail("driver value '" + name + "' is not declared");
        return it->second;
    }

    // ------------------------------------------------------------------------ compiling drivers

    void compile(Entry & e) {
        e.code.clear();
        emit_code(e.code, e.spec->driver);
    }

    void emit_code(std::vector<VmCode> & code, const std::vector<DriverOp> & ops_) {
        for (const DriverOp & d : ops_) {
            if (!d.loop) {
                code.push_back({VmCode::Call, &d, -1, call_for(d)});
                continue;
            }
            check_loop(d);
            code.push_back({VmCode::Enter, &d, -1, -1});
            const int top = (int) code.size();
            code.push_back({VmCode::Top, &d, -1, -1});
            emit_code(code, d.body);
            code.push_back({VmCode::Bottom, &d, top, -1});
            code[(size_t) top].jump = (int) code.size();
        }
    }

    void check_loop(const DriverOp & d) const {
        for (const auto & c : d.carry) {
            const ggml_tensor *a = value(c.first), *b = value(c.second);
            if (a->type != b->type || !ggml_are_same_shape(a, b))
                fail("loop carry '" + c.first + "' does not match its initial value '" + c.second + "'");
        }
        for (const auto & sc : d.scalars)
            if (value(sc.first)->type != GGML_TYPE_F32) fail("loop scalar '" + sc.first + "' must be f32");
        for (const auto & sl : d.slices) {
            // the source is [n, ...row] in PyTorch order: the row's elements n times, outermost
            const ggml_tensor *row = value(sl.first), *src = value(sl.second);
            if (row->type != src->type || ggml_nelements(src) != ggml_nelements(row) * d.n || !ggml_is_contiguous(src) ||
                !ggml_is_contiguous(row))
                fail("loop slice '" + sl.first + "' does not match its source '" + sl.second + "'");
        }
        for (const auto & m : d.masks)
            if (spec.at(m.first)->type != GGML_TYPE_F32) fail("loop mask '" + m.first + "' must be f32");
    }

    // The call graph of driver call d, made the first time the call is compiled.
    int call_for(const DriverOp & d) {
        for (size_t k = 0; k < calls.size(); k++)
            if (calls[k].op == &d) return (int) k;
        CallGraph c;
        c.op = &d;
        for (size_t k = 0; k < prog.stages.size(); k++)
            if (prog.stages[k].name == d.stage) c.stage = (int) k;
        if (c.stage < 0) fail("driver calls unknown stage '" + d.stage + "'");
        calls.push_back(c);
        build_graph(calls.back());
        return (int) calls.size() - 1;
    }

    // ------------------------------------------------------------------------- stage graphs

    // The stage's results as tensors of c.ctx: from a compiled builder, or node by node.
    std::vector<ggml_tensor *> stage_results(CallGraph & c, const StageSpec & st,
                                             std::unordered_map<std::string, ggml_tensor *> & env) {
        std::vector<ggml_tensor *> results;
        const auto custom = builders.find(st.name);
        if (custom != builders.end()) {
            ggml_compiler_stage_build b;
            b.ctx = c.ctx;
            b.backend = backend;
            b.wctx = wctx;
            b.binding = &binding;
            for (const auto & p : st.params) b.params.push_back(env.at(p.name));
            b.outputs.assign(st.outputs.size(), nullptr);
            if (custom->second(&b) != 0 || !b.error.empty())
                fail("builder for stage '" + st.name + "' failed: " + b.error);
            for (size_t k = 0; k < st.outputs.size(); k++) {
                ggml_tensor * t = b.outputs[k];
                if (!t) fail("builder for stage '" + st.name + "' left output " + std::to_string(k) + " unset");
                for (const auto & nd : st.nodes) {
                    if (nd.id != st.outputs[k]) continue;
                    bool same = t->type == nd.type;
                    for (int q = 0; q < 4; q++) same = same && t->ne[q] == nd.ne[q];
                    if (!same)
                        fail("builder for stage '" + st.name + "' output " + std::to_string(k) +
                             " does not match the program");
                }
                results.push_back(t);
            }
            return results;
        }
        std::vector<ggml_tensor *> srcs;
        for (const auto & nd : st.nodes) {
            srcs.clear();
            for (const auto & name : nd.src) {
                const auto it = env.find(name);
                ggml_tensor * t = it != env.end() ? it->second : (wctx ? ggml_get_tensor(wctx, name.c_str()) : nullptr);
                if (!t) fail("stage '" + st.name + "' node " + nd.id + " reads unknown tensor '" + name + "'");
                srcs.push_back(t);
            }
            env[nd.id] = emit_node(c.ctx, nd, srcs);
        }
        for (const auto & id : st.outputs) {
            const auto it = env.find(id);
            if (it == env.end()) fail("stage '" + st.name + "' returns unknown value '" + id + "'");
            results.push_back(it->second);
        }
        return results;
    }

    void build_graph(CallGraph & c) {
        const StageSpec & st = prog.stages[(size_t) c.stage];
        const DriverOp & d = *c.op;
        if (d.args.size() != st.params.size() || d.out.size() != st.outputs.size())
            fail("call to stage '" + st.name + "' has the wrong number of arguments or results");
        const size_t tensors = 8 * st.nodes.size() + 2 * st.outputs.size() + 16;
        const size_t graph_nodes = tensors + st.params.size() + file.tensors.size() + 64;
        ggml_init_params ip{};
        ip.mem_size = ggml_tensor_overhead() * tensors + 2 * ggml_graph_overhead_custom(graph_nodes, false);
        ip.no_alloc = true;
        c.ctx = ggml_init(ip);
        std::unordered_map<std::string, ggml_tensor *> env;
        for (size_t k = 0; k < st.params.size(); k++) {
            ggml_tensor * arg = value(d.args[k]);
            const TensorSpec & p = st.params[k];
            bool fits = arg->type == p.type;
            for (int q = 0; q < 4; q++) fits = fits && arg->ne[q] == p.ne[q];
            if (!fits) fail("stage '" + st.name + "' parameter " + p.name + " does not match value '" + d.args[k] + "'");
            env[p.name] = arg;
        }
        const std::vector<ggml_tensor *> results = stage_results(c, st, env);
        c.graph = ggml_new_graph_custom(c.ctx, graph_nodes, false);
        // get_rows / copies that read only the stage's parameters and weights (an embedding row, a
        // mask's cast) come first, in their order, so that the executor can run such small steps
        // together in one launch. Moving a node changes nothing only if no other node writes what
        // it reads or reads what it writes: a leaf written in place (set_rows' destination, a copy's
        // destination) keeps its nodes in the expand order, as ggml would run them.
        ggml_cgraph * probe = ggml_new_graph_custom(c.ctx, graph_nodes, false);
        for (ggml_tensor * t : results) ggml_build_forward_expand(probe, t);
        auto leaf_of = [](const ggml_tensor * t) {
            while (t && (t->op == GGML_OP_VIEW || t->op == GGML_OP_RESHAPE || t->op == GGML_OP_PERMUTE ||
                         t->op == GGML_OP_TRANSPOSE))
                t = t->src[0];
            return t;
        };
        auto dest_of = [&](const ggml_tensor * t) -> const ggml_tensor * {
            if (t->op == GGML_OP_SET_ROWS) return leaf_of(t->src[2]);
            if (t->op == GGML_OP_CPY) return leaf_of(t->src[1]);
            return nullptr;
        };
        std::unordered_map<const ggml_tensor *, int> writers, readers;
        for (int k = 0; k < ggml_graph_n_nodes(probe); k++) {
            const ggml_tensor * t = ggml_graph_node(probe, k);
            if (const ggml_tensor * d = dest_of(t)) writers[d]++;
            for (const ggml_tensor * src : t->src)
                if (src && src != (t->op == GGML_OP_CPY ? t->src[1] : nullptr)) readers[leaf_of(src)]++;
        }
        for (int k = 0; k < ggml_graph_n_nodes(probe); k++) {
            ggml_tensor * t = ggml_graph_node(probe, k);
            if (t->op != GGML_OP_GET_ROWS && t->op != GGML_OP_CPY) continue;
            bool movable = true;  // every source a leaf (or a view of one) nothing writes in place
            for (const ggml_tensor * src : t->src) {
                if (!src || (t->op == GGML_OP_CPY && src == t->src[1])) continue;
                const ggml_tensor * l = leaf_of(src);
                movable = movable && l->op == GGML_OP_NONE && writers.count(l) == 0;
            }
            if (const ggml_tensor * d = dest_of(t))  // a copy: its destination written and read by it alone
                movable = movable && writers[d] == 1 && readers.count(d) == 0;
            if (movable) ggml_build_forward_expand(c.graph, t);
        }
        for (ggml_tensor * t : results) ggml_build_forward_expand(c.graph, t);
        // Results reach their driver values through copies after every other node (so after
        // every read of the stage's arguments); a result that already is its value's memory (a
        // set_rows into the cache the stage read) needs none.
        for (size_t k = 0; k < results.size(); k++) {
            ggml_tensor *dst = value(d.out[k]), *res = results[k];
            const bool in_place = res == dst || (res->data && res->data == dst->data && res->type == dst->type &&
                                                 ggml_are_same_shape(res, dst) && ggml_is_contiguous(res));
            if (in_place) continue;
            if (ggml_nelements(res) != ggml_nelements(dst) || res->type != dst->type)
                fail("stage '" + st.name + "' result " + std::to_string(k) + " does not match value '" + d.out[k] + "'");
            ggml_build_forward_expand(c.graph, ggml_cpy(c.ctx, res, dst));
        }
        std::string refused;
        for (int k = 0; k < ggml_graph_n_nodes(c.graph); k++) {
            ggml_tensor * t = ggml_graph_node(c.graph, k);
            if (!ggml_backend_supports_op(backend, t))
                refused += std::string("\n  ") + t->name + " (" + ggml_op_desc(t) + "): " + last_error();
        }
        if (!refused.empty())
            fail(std::string("backend ") + ggml_backend_name(backend) + " cannot run these nodes of stage '" + st.name +
                 "':" + refused);
        const bool symbolic = prog.stages[(size_t) c.stage].symbolic;
        if (symbolic || !c.alloc) c.alloc = ggml_gallocr_new(ggml_backend_get_default_buffer_type(backend));
        if (!ggml_gallocr_alloc_graph(c.alloc, c.graph))
            fail("cannot allocate compute buffer for stage '" + st.name + "': " + last_error());
        if (symbolic) c.builds.push_back({binding, c.ctx, c.graph, c.alloc});
        c.stale = false;
    }

    // A new binding: values viewed at their new shapes; stages whose shapes read a symbol use their
    // graph of this binding, or build one when next run (so an entry never builds another entry's
    // stages).
    void apply_binding() {
        if (binding == built) return;
        prog.bind(binding);
        make_views();
        for (auto & c : calls) {
            if (!prog.stages[(size_t) c.stage].symbolic) continue;
            c.ctx = nullptr, c.graph = nullptr, c.alloc = nullptr, c.stale = true;
            for (const CallGraph::Build & b : c.builds)
                if (b.binding == binding) c.use(b);
        }
        for (auto & e : entries)
            for (const VmCode & vc : e.code)
                if (vc.kind == VmCode::Enter) check_loop(*vc.op);
        built = binding;
    }

    // ------------------------------------------------------------------------------- running

    void run_call(CallGraph & c) {
        ops.flush();  // the driver's waiting ops before the stage's graph
        if (c.stale) build_graph(c);
        const StageSpec & st = prog.stages[(size_t) c.stage];
        last.n_calls++;
        if (profile_file()) {
            run_nodes(c, st);
            return;
        }
        clock.before(ops.stream());
        if (graph_compute_async(backend, c.graph) != GGML_STATUS_SUCCESS)
            fail("stage '" + st.name + "' failed: " + last_error());
        clock.after(c.stage, ops.stream(), cur_group);
    }

    // Profiling: each node of the graph alone, waited for and timed.
    void run_nodes(CallGraph & c, const StageSpec & st) {
        using wall = std::chrono::steady_clock;
        const auto t_call = wall::now();
        ggml_cgraph one;
        for (int k = 0; k < ggml_graph_n_nodes(c.graph); k++) {
            ggml_tensor * t = ggml_graph_node(c.graph, k);
            one.nodes.assign(1, t);
            const auto t0 = wall::now();
            if (ggml_backend_graph_compute(backend, &one) != GGML_STATUS_SUCCESS)
                fail("profiling: node " + std::string(t->name) + " of stage '" + st.name + "' failed: " + last_error());
            profile.push_back({st.name, t->name, ggml_op_desc(t),
                               std::chrono::duration<double, std::milli>(wall::now() - t0).count()});
        }
        auto & tot = stage_totals[(size_t) c.stage];
        tot.ms_total += std::chrono::duration<double, std::milli>(wall::now() - t_call).count();
        tot.n_calls++;
    }

    void loop_enter(LoopFrame & f) {
        const DriverOp & d = *f.op;
        for (const auto & c : d.carry) ops.copy(value(c.first)->data, value(c.second)->data, ggml_nbytes(value(c.first)));
        f.trips = d.n_symbol >= 0 ? (int) binding[(size_t) d.n_symbol] : d.n;
        f.i = 0;
        f.start.clear();
        for (const auto & c : d.counters) f.start.push_back(ops.read_i32(value(c.second)->data));
        for (const auto & c : d.collect) {
            ggml_tensor * t = storage.at(c.first);
            ops.clear(t->data, ggml_nbytes(t));
        }
        f.cap = loop_state(d);
        f.until = f.cap && f.cap->has_until ? f.cap : nullptr;
        if (f.cap) {
            ops.fill32(f.cap->it, 1, 0u);
            ops.fill32(f.cap->stop, 1, (uint32_t) INT32_MAX);  // no stop yet (or ever, without an until test)
            for (size_t k = 0; k < f.start.size() && k < (size_t) kUntilCounters; k++)
                ops.fill32(f.cap->base + k, 1, (uint32_t) f.start[k]);
        }
        if (f.until) {
            // the loop's previous run waited for its last test op, so nothing still writes these
            __atomic_store_n(&f.until->host[0], INT32_MAX, __ATOMIC_RELAXED);
            __atomic_store_n(&f.until->host[1], 0, __ATOMIC_RELEASE);
        }
    }

    // The device state of loop d, for a body of calls only: its iterations can be captured and
    // replayed (UntilState), and its until test, if it has one of one i32 value whose body's values
    // (state aside) take at most kUntilKeepMax bytes, runs on the device. Other loops (and every
    // loop when profiling node by node) run uncaptured and read their until values after every
    // iteration. Made on the loop's first entry.
    static constexpr size_t kUntilKeepMax = 16u << 20;
    UntilState * loop_state(const DriverOp & d) {
        if (profile_file()) return nullptr;
        auto it = untils.find(&d);
        if (it != untils.end()) return it->second.get();
        const bool dev_until = d.until.size() == 1 && spec.at(d.until[0].first)->type == GGML_TYPE_I32;
        if (!d.until.empty() && !dev_until) {
            if (log_debug()) std::fprintf(stderr, "ggml_compiler: loop runs uncaptured: its until test is not one i32 value\n");
            return nullptr;
        }
        std::vector<std::string> kept;
        auto keep = [&](const std::string & v) {
            if (std::find(prog.state.begin(), prog.state.end(), v) == prog.state.end() &&
                std::find(kept.begin(), kept.end(), v) == kept.end())
                kept.push_back(v);
        };
        for (const DriverOp & b : d.body) {
            if (b.loop) {
                if (log_debug()) std::fprintf(stderr, "ggml_compiler: loop runs uncaptured: its body holds a loop\n");
                return nullptr;
            }
            for (const auto & v : b.out) keep(v);
        }
        for (const auto & c : d.carry) keep(c.first);
        if (!dev_until) kept.clear();  // the ring serves the until test's roll-back only
        auto u = std::make_unique<UntilState>();
        u->has_until = dev_until;
        const std::vector<int> ids = dev_until ? d.until[0].second : std::vector<int>{};
        size_t keep_bytes = 0;
        for (const auto & v : kept) {
            u->slot_bytes.push_back(align256(ggml_nbytes(storage.at(v))));
            keep_bytes += 2 * u->slot_bytes.back();
        }
        if (keep_bytes > kUntilKeepMax) {
            if (log_debug()) std::fprintf(stderr, "ggml_compiler: loop runs uncaptured: %zu bytes to keep\n", keep_bytes);
            return nullptr;
        }
        u->kept = kept;
        const size_t id_bytes = align256(std::max<size_t>(1, ids.size()) * 4);
        check_hip(hipMalloc(&u->dev, 256 + id_bytes + keep_bytes), "hipMalloc (until)");
        check_hip(hipHostMalloc((void **) &u->host, 2 * sizeof(int32_t), hipHostMallocCoherent), "hipHostMalloc (until)");
        uint8_t * p = (uint8_t *) u->dev;
        u->stop = (int32_t *) p;
        u->it = (int32_t *) p + 1;
        u->base = (int32_t *) p + 2;
        u->ids = (int32_t *) (p + 256);
        u->n_ids = (int64_t) ids.size();
        uint8_t * r = p + 256 + id_bytes;
        for (size_t k = 0; k < kept.size(); k++) {
            u->ring.push_back(r);
            r += 2 * u->slot_bytes[k];
        }
        std::vector<int32_t> id32(ids.begin(), ids.end());
        if (!id32.empty())
            check_hip(hipMemcpy(u->ids, id32.data(), id32.size() * 4, hipMemcpyHostToDevice), "until ids");
        // captured iterations: the scalars' values per iteration on the device
        u->group = (int) untils.size();
        u->graphable = d.counters.size() <= (size_t) kUntilCounters && !d.body.empty();
        size_t tab_bytes = 0;
        for (const auto & sc : d.scalars) tab_bytes += align256(std::max<size_t>(1, sc.second.size()) * 4);
        if (u->graphable && tab_bytes) {
            check_hip(hipMalloc(&u->tab_mem, tab_bytes), "hipMalloc (loop scalars)");
            uint8_t * t = (uint8_t *) u->tab_mem;
            for (const auto & sc : d.scalars) {
                if (!sc.second.empty())
                    check_hip(hipMemcpy(t, sc.second.data(), sc.second.size() * 4, hipMemcpyHostToDevice), "loop scalars");
                u->tabs.push_back((const uint32_t *) t);
                t += align256(std::max<size_t>(1, sc.second.size()) * 4);
            }
        }
        UntilState * raw = u.get();
        untils.emplace(&d, std::move(u));
        return raw;
    }

    // Waits until the device's until test has run for `done` iterations of the loop (the test op
    // writes the host's copy; the GPU keeps the next iteration queued meanwhile).
    void wait_tested(const UntilState & u, int32_t done) {
        unsigned spins = 0;
        while (__atomic_load_n(&u.host[1], __ATOMIC_ACQUIRE) < done) {
            if ((++spins & 1023u) == 0u) {
                const hipError_t q = hipStreamQuery(ops.stream());
                if (q == hipSuccess) {
                    if (__atomic_load_n(&u.host[1], __ATOMIC_ACQUIRE) >= done) break;
                    fail("loop: the until test of iteration " + std::to_string(done - 1) + " did not report");
                }
                if (q != hipErrorNotReady) check_hip(q, "loop until test");
            }
            std::this_thread::yield();
        }
    }

    // Before the body of iteration f.i: scalars, slices, counters, bound symbols, causal masks.
    void loop_top(LoopFrame & f) {
        const DriverOp & d = *f.op;
        const int i = f.i;
        for (const auto & sc : d.scalars) {
            ggml_tensor * t = value(sc.first);
            uint32_t bits;
            std::memcpy(&bits, &sc.second[(size_t) i], 4);
            ops.fill32(t->data, ggml_nelements(t), bits);
        }
        for (const auto & sl : d.slices) {
            ggml_tensor *row = value(sl.first), *src = value(sl.second);
            const size_t nb = ggml_nbytes(row);
            ops.copy(row->data, (const char *) src->data + (size_t) i * nb, nb);
        }
        for (size_t k = 0; k < d.counters.size(); k++)
            ops.fill32(value(d.counters[k].first)->data, 1, (uint32_t) (f.start[k] + i));
        if (!d.bind.empty()) {
            std::vector<int64_t> with_counters = binding;
            for (int32_t v : f.start) with_counters.push_back(v + i);
            for (const auto & bnd : d.bind) {
                const int64_t v = bnd.second(with_counters);
                const Symbol & sy = prog.symbols[(size_t) bnd.first];
                if (v < sy.min || v > sy.max)
                    fail("loop binds " + sy.name + " = " + std::to_string(v) + ", outside its range");
                binding[(size_t) bnd.first] = v;
            }
            apply_binding();
        }
        for (const auto & m : d.masks) {
            const TensorSpec & v = *spec.at(m.first);
            ops.causal((float *) storage.at(m.first)->data, v.ne[0] * v.ne[1] * v.ne[2] * v.ne[3], v.ne[0],
                       f.start[(size_t) m.second] + i);
        }
    }

    // After the body: collected rows; true when an until value holds a stop id.
    bool loop_bottom(LoopFrame & f) {
        const DriverOp & d = *f.op;
        if (f.until) return loop_bottom_device(f);
        if (f.replayed) {  // its graph holds the collects; the loop has no until test
            f.replayed = false;
            return false;
        }
        for (const auto & c : d.collect) {
            const size_t nb = spec.at(c.second)->nbytes(binding);
            ops.copy((char *) storage.at(c.first)->data + (size_t) f.i * nb, storage.at(c.second)->data, nb);
        }
        if (f.cap) ops.fill32(f.cap->it, 1, (uint32_t) (f.i + 1));  // the iteration word, for a replay of the next
        for (const auto & u : d.until) {
            const int32_t tok = ops.read_i32(storage.at(u.first)->data);
            if (std::find(u.second.begin(), u.second.end(), tok) != u.second.end()) return true;
        }
        return false;
    }

    // loop_bottom with the until test on the device. Iteration i's row is collected only at or
    // before the stop, its test op sets the stop word and the host's copy, and the values its body
    // wrote (state aside) go to a ring slot. The host then checks iteration i - 1's test
    // (iteration i stays queued on the GPU meanwhile, so no iteration waits for the host): when
    // i - 1 stopped, iteration i ran past the loop's end, and every value the loop leaves
    // (loop-top values, the body's results, carries) is put back to iteration i - 1's, and the
    // stats drop iteration i's calls. Its one other effect is on state: what the body writes
    // there one iteration past the stop (the K / V row of the next position, which a later
    // decode of that position writes before any read). True when the loop ends.
    bool loop_bottom_device(LoopFrame & f) {
        const DriverOp & d = *f.op;
        UntilState & u = *f.until;
        const int i = f.i;
        if (!f.replayed) {  // a replayed iteration's graph holds these ops
            for (const auto & c : d.collect) {
                const size_t nb = spec.at(c.second)->nbytes(binding);
                ops.copy_if((char *) storage.at(c.first)->data + (size_t) i * nb, storage.at(c.second)->data, nb, u.stop, i);
            }
            ops.until((const int32_t *) storage.at(d.until[0].first)->data, u.ids, u.n_ids, u.stop, u.host, i);
            for (size_t k = 0; k < u.kept.size(); k++) {
                ggml_tensor * v = value(u.kept[k]);
                ops.copy(u.ring[k] + (size_t) (i & 1) * u.slot_bytes[k], v->data, ggml_nbytes(v));
            }
            ops.fill32(u.it, 1, (uint32_t) (i + 1));  // the iteration word, for a replay of the next
        }
        f.replayed = false;
        ops.flush();
        if (i >= 1) {
            wait_tested(u, i);
            const int32_t stop = __atomic_load_n(&u.host[0], __ATOMIC_RELAXED);
            if (stop <= i - 1) {
                last.n_calls = f.calls0;  // the stats count the calls of the loop's iterations only
                clock.forget_since(f.marks0);
                f.i = stop;
                loop_top(f);  // iteration `stop`'s scalars, slices, counters, symbols, masks
                for (size_t k = 0; k < u.kept.size(); k++) {
                    ggml_tensor * v = value(u.kept[k]);
                    ops.copy(v->data, u.ring[k] + (size_t) (stop & 1) * u.slot_bytes[k], ggml_nbytes(v));
                }
                wait_tested(u, i + 1);  // nothing of the loop writes the host's copy after this
                return true;
            }
        }
        if (i + 1 >= f.trips) {
            wait_tested(u, i + 1);
            return true;
        }
        return false;
    }

    // The binding of the symbols that iteration f.i binds (loop_top's rule), without applying it.
    std::vector<int64_t> bind_for(const LoopFrame & f) const {
        std::vector<int64_t> b = binding, with = binding;
        for (int32_t v : f.start) with.push_back(v + f.i);
        for (const auto & bnd : f.op->bind) b[(size_t) bnd.first] = bnd.second(with);
        return b;
    }

    // Iteration f.i of a loop with a device until test, replayed from the loop's captured graph
    // (captured now if there is none for the current binding): when it is not the loop's first
    // iteration and binds the symbols as the previous one did (whose uncaptured run planned the
    // stages' graphs for them), and every iteration copy fits one driver op. False: run it
    // uncaptured.
    bool replay_iteration(LoopFrame & f, const std::vector<VmCode> & code, size_t top) {
        f.replayed = false;
        UntilState * u = f.cap;
        if (!u || !u->graphable || f.i < 1 || profile_file()) return false;
        const DriverOp & d = *f.op;
        auto no = [&](const char * why) {
            if (log_debug()) std::fprintf(stderr, "ggml_compiler: loop iteration %d uncaptured: %s\n", f.i, why);
            return false;
        };
        if (!d.bind.empty() && bind_for(f) != binding) return no("binding changed");
        for (const auto & sl : d.slices)
            if (ggml_nbytes(value(sl.first)) > kDriverCopyMax) return no("slice too large");
        for (const auto & c : d.collect)
            if (spec.at(c.second)->nbytes(binding) > kDriverCopyMax) return no("collect too large");
        for (const auto & k : u->kept)
            if (ggml_nbytes(value(k)) > kDriverCopyMax) return no("kept value too large");
        for (size_t k = top + 1; code[k].kind == VmCode::Call; k++)
            if (calls[(size_t) code[k].call].stale) return no("stage graph stale");
        const uint64_t epoch = backend_epoch(backend);
        UntilState::IterGraph * g = nullptr;
        for (auto & ig : u->graphs)
            if (ig.binding == binding) g = &ig;
        if (g && g->epoch != epoch) {
            u->drop_graphs(&binding);
            g = nullptr;
        }
        if (!g) {
            hipGraphExec_t exec = nullptr;
            try {
                exec = capture_iteration(f, code, top);
            } catch (const Fail & e) {  // not capturable: this loop runs uncaptured from now on
                u->graphable = false;
                if (log_debug()) std::fprintf(stderr, "ggml_compiler: loop iteration not captured: %s\n", e.msg.c_str());
                return false;
            }
            if (log_debug()) std::fprintf(stderr, "ggml_compiler: loop iteration %d captured\n", f.i);
            u->graphs.push_back({binding, epoch, exec});
            g = &u->graphs.back();
        }
        const hipStream_t s = ops.stream();
        clock.before(s);
        check_hip(hipGraphLaunch(g->exec, s), "hipGraphLaunch (loop iteration)");
        clock.after_iteration(u->group, &u->body_stages, s);
        last.n_calls += u->body_stages.size();
        f.replayed = true;
        return true;
    }

    // One iteration of the loop at `top` captured into a graph: its top ops, the body's stage
    // graphs as plain launches (the executor's own graph capture off meanwhile), its bottom ops and
    // the step of the iteration word, all in iteration-relative form.
    hipGraphExec_t capture_iteration(LoopFrame & f, const std::vector<VmCode> & code, size_t top) {
        UntilState & u = *f.cap;
        const hipStream_t s = ops.stream();  // every waiting op launched, before the capture
        std::vector<int> stages;
        hipGraph_t graph = nullptr;
        ggml_backend_hip_set_use_graphs(backend, false);
        const hipError_t b = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
        if (b != hipSuccess) {
            ggml_backend_hip_set_use_graphs(backend, true);
            (void) hipGetLastError();
            fail(std::string("hipStreamBeginCapture: ") + hipGetErrorString(b));
        }
        try {
            loop_top_rel(f);
            for (size_t k = top + 1; code[k].kind == VmCode::Call; k++) {
                CallGraph & c = calls[(size_t) code[k].call];
                ops.flush();
                if (graph_compute_async(backend, c.graph) != GGML_STATUS_SUCCESS)
                    fail("stage '" + prog.stages[(size_t) c.stage].name + "' failed: " + last_error());
                stages.push_back(c.stage);
            }
            loop_bottom_rel(f);
            ops.iter_next(u.it);
        } catch (...) {
            ops.discard();
            (void) hipStreamEndCapture(s, &graph);
            if (graph) (void) hipGraphDestroy(graph);
            (void) hipGetLastError();
            ggml_backend_hip_set_use_graphs(backend, true);
            throw;
        }
        const hipError_t e1 = hipStreamEndCapture(s, &graph);
        ggml_backend_hip_set_use_graphs(backend, true);
        if (e1 != hipSuccess) {
            if (graph) (void) hipGraphDestroy(graph);
            (void) hipGetLastError();
            fail(std::string("hipStreamEndCapture: ") + hipGetErrorString(e1));
        }
        hipGraphExec_t exec = nullptr;
        const hipError_t e2 = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void) hipGraphDestroy(graph);
        check_hip(e2, "hipGraphInstantiate (loop iteration)");
        u.body_stages = std::move(stages);
        return exec;
    }

    // loop_top's ops in iteration-relative form (the binding is the current one).
    void loop_top_rel(LoopFrame & f) {
        const DriverOp & d = *f.op;
        const UntilState & u = *f.cap;
        for (size_t k = 0; k < d.scalars.size(); k++) {
            ggml_tensor * t = value(d.scalars[k].first);
            ops.fill32_tab(t->data, ggml_nelements(t), u.tabs[k], u.it);
        }
        for (const auto & sl : d.slices) {
            ggml_tensor *row = value(sl.first), *src = value(sl.second);
            const size_t nb = ggml_nbytes(row);
            ops.copy_rel(row->data, src->data, nb, 0, (int64_t) nb, false, u.it, nb, ggml_nbytes(src));
        }
        for (size_t k = 0; k < d.counters.size(); k++)
            ops.fill32_ctr(value(d.counters[k].first)->data, 1, u.base + k, u.it);
        for (const auto & m : d.masks) {
            const TensorSpec & v = *spec.at(m.first);
            ops.causal_rel((float *) storage.at(m.first)->data, v.ne[0] * v.ne[1] * v.ne[2] * v.ne[3], v.ne[0],
                           u.base + m.second, u.it);
        }
    }

    // loop_bottom's ops in iteration-relative form (without an until test the collects are
    // unconditional: the stop word stays INT32_MAX).
    void loop_bottom_rel(LoopFrame & f) {
        const DriverOp & d = *f.op;
        UntilState & u = *f.cap;
        for (const auto & c : d.collect) {
            const size_t nb = spec.at(c.second)->nbytes(binding);
            ggml_tensor * dst = storage.at(c.first);
            ops.copy_if_rel(dst->data, storage.at(c.second)->data, nb, (int64_t) nb, u.stop, u.it, ggml_nbytes(dst));
        }
        if (u.has_until)
            ops.until_rel((const int32_t *) storage.at(d.until[0].first)->data, u.ids, u.n_ids, u.stop, u.host, u.it);
        for (size_t k = 0; k < u.kept.size(); k++) {
            ggml_tensor * v = value(u.kept[k]);
            ops.copy_rel(u.ring[k], v->data, ggml_nbytes(v), (int64_t) u.slot_bytes[k], 0, true, u.it,
                         2 * u.slot_bytes[k], ggml_nbytes(v));
        }
    }

    void execute(const Entry & e) {
        std::vector<LoopFrame> frames;
        const std::vector<VmCode> & code = e.code;
        size_t pc = 0;
        while (pc < code.size()) {
            const VmCode & in = code[pc];
            switch (in.kind) {
                case VmCode::Call:
                    run_call(calls[(size_t) in.call]);
                    pc++;
                    break;
                case VmCode::Enter:
                    frames.push_back({in.op, 0, 0, {}, nullptr});
                    loop_enter(frames.back());
                    pc++;
                    break;
                case VmCode::Top:
                    if (frames.back().i >= frames.back().trips) {
                        frames.pop_back();
                        cur_group = -1;
                        pc = (size_t) in.jump;
                    } else {
                        LoopFrame & f = frames.back();
                        f.calls0 = last.n_calls;
                        f.marks0 = clock.marks();
                        cur_group = f.cap ? f.cap->group : -1;
                        if (replay_iteration(f, code, pc)) {
                            pc = (size_t) in.jump - 1;  // the loop's Bottom
                        } else {
                            loop_top(f);
                            pc++;
                        }
                    }
                    break;
                case VmCode::Bottom:
                    if (loop_bottom(frames.back())) {
                        frames.pop_back();
                        cur_group = -1;
                        pc = (size_t) code[(size_t) in.jump].jump;
                    } else {
                        frames.back().i++;
                        pc = (size_t) in.jump;
                    }
                    break;
            }
        }
    }

    void run(const char * entry_name) {
        const Entry * e = nullptr;
        for (const auto & en : entries)
            if (en.spec->name == entry_name) e = &en;
        require(e != nullptr, "no entry point named '" + std::string(entry_name) + "'");
        for (const TensorSpec * v : e->in) require(inputs_set.count(v->name) != 0, "input '" + v->name + "' was never set");
        apply_binding();
        for (auto & t : stage_totals) t = ggml_compiler_stats{};
        last = ggml_compiler_stats{};
        ops.discard();
        clock.begin_run();
        const auto t0 = std::chrono::steady_clock::now();
        execute(*e);
        ops.finish();
        last.ms_total = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        clock.collect([&](int stage, double ms, int n) {
            stage_totals[(size_t) stage].ms_total += ms;
            stage_totals[(size_t) stage].n_calls += n;
        });
        write_profile();
    }

    void write_profile() {
        if (!profile_file() || profile.empty()) return;
        if (FILE * f = std::fopen(profile_file(), "a")) {
            for (const auto & p : profile)
                std::fprintf(f, "%s\t%s\t%s\t%.6f\n", p.stage.c_str(), p.node.c_str(), p.op.c_str(), p.ms);
            std::fclose(f);
        }
        profile.clear();
    }

    // ------------------------------------------------------------------------- inputs, outputs

    const TensorSpec & input(const char * name) const {
        for (const auto & e : entries)
            for (const TensorSpec * v : e.in)
                if (v->name == name) return *v;
        fail("no input named '" + std::string(name) + "'");
    }

    // The symbols an input's shape fixes: a dim with one unknown symbol is solved by bisection over
    // the symbol's range (dims are monotone in each symbol); then every dim must match.
    void bind_shape(const TensorSpec & v, const std::vector<int64_t> & shape) {
        if (shape.size() != v.shape_x.size())
            fail("input '" + v.name + "' has rank " + std::to_string(v.shape_x.size()) + ", got " +
                 std::to_string(shape.size()));
        std::vector<int64_t> b = binding;
        std::vector<bool> known(b.size(), false);
        for (int pass = 0; pass < 2; pass++) {
            for (size_t i = 0; i < shape.size(); i++) {
                std::vector<bool> used(b.size(), false);
                v.shape_x[i].mark(used);
                int unknown = -1, n_unknown = 0;
                for (size_t k = 0; k < used.size(); k++)
                    if (used[k] && !known[k]) {
                        unknown = (int) k;
                        n_unknown++;
                    }
                if (n_unknown != 1) continue;
                const Symbol & sy = prog.symbols[(size_t) unknown];
                int64_t lo = sy.min, hi = sy.max;
                while (lo < hi) {  // the smallest value whose dim reaches shape[i]
                    const int64_t mid = lo + (hi - lo) / 2;
                    b[(size_t) unknown] = mid;
                    if (v.shape_x[i](b) < shape[i]) lo = mid + 1;
                    else hi = mid;
                }
                b[(size_t) unknown] = lo;
                if (v.shape_x[i](b) != shape[i])
                    fail("input '" + v.name + "': no " + sy.name + " in [" + std::to_string(sy.min) + ", " +
                         std::to_string(sy.max) + "] gives dim " + std::to_string(i) + " = " + std::to_string(shape[i]));
                known[(size_t) unknown] = true;
            }
        }
        const std::vector<int64_t> got = v.shape(b);
        if (got != shape) {
            std::string want, have;
            for (auto dv : shape) want += (want.empty() ? "" : ", ") + std::to_string(dv);
            for (auto dv : got) have += (have.empty() ? "" : ", ") + std::to_string(dv);
            fail("input '" + v.name + "' cannot have shape [" + want + "] (with the other symbols as bound, it is [" +
                 have + "])");
        }
        binding = b;
    }

    void write_input(const char * name, const void * data, size_t nbytes) {
        const TensorSpec & v = input(name);
        const size_t want = v.nbytes(binding);
        require(nbytes == want, "input '" + std::string(name) + "' needs " + std::to_string(want) + " bytes, got " +
                                    std::to_string(nbytes));
        ggml_checked("input '" + std::string(name) + "'",
                     [&] { ggml_backend_tensor_set(storage.at(v.name), data, 0, nbytes); });
        inputs_set.insert(v.name);
    }

    void read_output(const char * name, void * dst, size_t nbytes) const {
        for (const auto & e : entries)
            for (const TensorSpec * v : e.out) {
                if (v->name != name) continue;
                const size_t have = v->nbytes(built);
                require(nbytes == have, "output '" + std::string(name) + "' has " + std::to_string(have) +
                                            " bytes, buffer has " + std::to_string(nbytes));
                ggml_checked("output '" + std::string(name) + "'",
                             [&] { ggml_backend_tensor_get(storage.at(name), dst, 0, nbytes); });
                return;
            }
        fail("no output named '" + std::string(name) + "'");
    }

    void clear_state() {
        for (const auto & name : prog.state) {
            ggml_tensor * t = storage.at(name);
            ops.clear(t->data, ggml_nbytes(t));
        }
        ops.finish();
    }

    void describe(const TensorSpec & v, const std::vector<int64_t> & b, ggml_compiler_tensor_info * info) const {
        require(info != nullptr, "info is NULL");
        static const std::map<int, ggml_compiler_dtype> dtypes = {
            {GGML_TYPE_F32, GGML_COMPILER_DTYPE_F32}, {GGML_TYPE_F16, GGML_COMPILER_DTYPE_F16},
            {GGML_TYPE_I32, GGML_COMPILER_DTYPE_I32}};
        const auto dt = dtypes.find(v.type);
        if (dt == dtypes.end()) fail("value '" + v.name + "' has a type the C API cannot describe");
        const std::vector<int64_t> shape = v.shape(b);
        require(shape.size() <= GGML_COMPILER_MAX_RANK, "value '" + v.name + "' has rank above GGML_COMPILER_MAX_RANK");
        info->name = v.name.c_str();
        info->dtype = dt->second;
        info->ndim = (int) shape.size();
        std::copy(shape.begin(), shape.end(), info->shape);
        info->nbytes = v.nbytes(b);
    }

    const Entry * entry_at(int e) const { return e >= 0 && e < (int) entries.size() ? &entries[(size_t) e] : nullptr; }
};

// ------------------------------------------------------------------------------------ C API

namespace {

// A C entry point's body: 0, or -1 with the message recorded; pointer / value variants return
// `bad` on an error.
template <class F>
int api(F && f) {
    return guarded(std::forward<F>(f));
}
template <class T, class F>
T api_or(T bad, F && f) {
    T out = bad;
    return guarded([&] { out = f(); }) == 0 ? out : bad;
}

}  // namespace

extern "C" {

ggml_compiler_model * ggml_compiler_load(const char * path, const ggml_compiler_options * opt) {
    return ggml_compiler_load_with(path, opt, nullptr, 0);
}

ggml_compiler_model * ggml_compiler_load_with(const char * path, const ggml_compiler_options * opt,
                                              const ggml_compiler_builder * builders, int n_builders) {
    return api_or<ggml_compiler_model *>(nullptr, [&] {
        require(path != nullptr, "path is NULL");
        require(n_builders == 0 || builders != nullptr, "builders is NULL");
        auto m = std::make_unique<ggml_compiler_model>();
        for (int k = 0; k < n_builders; k++) {
            require(builders[k].stage && builders[k].build, "builder " + std::to_string(k) + " is incomplete");
            m->builders[builders[k].stage] = builders[k].build;
        }
        m->open(path, opt ? *opt : ggml_compiler_default_options());
        for (const auto & kv : m->builders) {
            const bool known = std::any_of(m->prog.stages.begin(), m->prog.stages.end(),
                                           [&](const StageSpec & st) { return st.name == kv.first; });
            if (!known) fail("builder for stage '" + kv.first + "', which the program does not have");
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
    if (i >= 0 && i < (int) b->params.size()) return b->params[(size_t) i];
    b->error = "parameter index " + std::to_string(i) + " out of range";
    return nullptr;
}

ggml_tensor * ggml_compiler_build_weight(ggml_compiler_stage_build * b, const char * name) {
    if (!b) return nullptr;
    ggml_tensor * t = (b->wctx && name) ? ggml_get_tensor(b->wctx, name) : nullptr;
    if (!t) b->error = std::string("no tensor '") + (name ? name : "(null)") + "' in the GGUF";
    return t;
}

int64_t ggml_compiler_build_symbol(ggml_compiler_stage_build * b, int i) {
    if (!b) return 1;
    if (b->binding && i >= 0 && i < (int) b->binding->size()) return (*b->binding)[(size_t) i];
    b->error = "symbol index " + std::to_string(i) + " out of range";
    return 1;
}

void ggml_compiler_build_output(ggml_compiler_stage_build * b, int i, ggml_tensor * t) {
    if (!b) return;
    if (i >= 0 && i < (int) b->outputs.size()) b->outputs[(size_t) i] = t;
    else b->error = "output index " + std::to_string(i) + " out of range";
}

const char * ggml_compiler_metadata(const ggml_compiler_model * m, const char * key) {
    if (!m || !key) return nullptr;
    const auto it = m->file.strings.find(key);
    return it == m->file.strings.end() ? nullptr : it->second.c_str();
}

void ggml_compiler_free(ggml_compiler_model * m) { delete m; }

const char * ggml_compiler_backend_name(const ggml_compiler_model * m) {
    return m ? ggml_backend_name(m->backend) : nullptr;
}

int ggml_compiler_n_entries(const ggml_compiler_model * m) { return m ? (int) m->entries.size() : -1; }

const char * ggml_compiler_entry_name(const ggml_compiler_model * m, int e) {
    const auto * en = m ? m->entry_at(e) : nullptr;
    if (en) return en->spec->name.c_str();
    set_error("entry index out of range");
    return nullptr;
}

int ggml_compiler_entry_n_inputs(const ggml_compiler_model * m, int e) {
    const auto * en = m ? m->entry_at(e) : nullptr;
    return en ? (int) en->in.size() : -1;
}

int ggml_compiler_entry_n_outputs(const ggml_compiler_model * m, int e) {
    const auto * en = m ? m->entry_at(e) : nullptr;
    return en ? (int) en->out.size() : -1;
}

int ggml_compiler_entry_input_info(const ggml_compiler_model * m, int e, int i, ggml_compiler_tensor_info * info) {
    return api([&] {
        const auto * en = m ? m->entry_at(e) : nullptr;
        require(en && i >= 0 && i < (int) en->in.size(), "input index out of range");
        m->describe(*en->in[(size_t) i], m->binding, info);
    });
}

int ggml_compiler_entry_output_info(const ggml_compiler_model * m, int e, int i, ggml_compiler_tensor_info * info) {
    return api([&] {
        const auto * en = m ? m->entry_at(e) : nullptr;
        require(en && i >= 0 && i < (int) en->out.size(), "output index out of range");
        m->describe(*en->out[(size_t) i], m->binding, info);
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
    return api([&] {
        require(m != nullptr, "model is NULL");
        m->clear_state();
    });
}

int ggml_compiler_n_symbols(const ggml_compiler_model * m) { return m ? (int) m->prog.symbols.size() : -1; }

int ggml_compiler_symbol_info(const ggml_compiler_model * m, int i, const char ** name, int64_t * min, int64_t * max,
                              int64_t * value) {
    return api([&] {
        require(m && i >= 0 && i < (int) m->prog.symbols.size(), "symbol index out of range");
        const Symbol & sy = m->prog.symbols[(size_t) i];
        if (name) *name = sy.name.c_str();
        if (min) *min = sy.min;
        if (max) *max = sy.max;
        if (value) *value = m->binding[(size_t) i];
    });
}

int ggml_compiler_set_symbol(ggml_compiler_model * m, const char * name, int64_t value) {
    return api([&] {
        require(m && name, "NULL argument");
        const int k = m->prog.symbol(name);
        require(k >= 0, "no symbol named '" + std::string(name) + "'");
        m->prog.check_range(k, value);
        m->binding[(size_t) k] = value;
    });
}

int ggml_compiler_set_input_shape(ggml_compiler_model * m, const char * name, int ndim, const int64_t * shape) {
    return api([&] {
        require(m && name && (ndim <= 0 || shape), "NULL argument");
        m->bind_shape(m->input(name), std::vector<int64_t>(shape, shape + std::max(ndim, 0)));
    });
}

int ggml_compiler_set_input(ggml_compiler_model * m, const char * name, const void * data, size_t nbytes) {
    return api([&] {
        require(m && name && data, "NULL argument");
        m->write_input(name, data, nbytes);
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
    return api([&] {
        require(m && entry, "NULL argument");
        m->run(entry);
    });
}

int ggml_compiler_get_output(ggml_compiler_model * m, const char * name, void * dst, size_t nbytes) {
    return api([&] {
        require(m && name && dst, "NULL argument");
        m->read_output(name, dst, nbytes);
    });
}

int ggml_compiler_last_stats(const ggml_compiler_model * m, ggml_compiler_stats * st) {
    return api([&] {
        require(m && st, "NULL argument");
        *st = m->last;
    });
}

int ggml_compiler_n_stages(const ggml_compiler_model * m) { return m ? (int) m->prog.stages.size() : -1; }

int ggml_compiler_stage_stats(const ggml_compiler_model * m, int i, const char ** name, double * ms, int * n_calls) {
    return api([&] {
        require(m && i >= 0 && i < (int) m->prog.stages.size(), "stage index out of range");
        if (name) *name = m->prog.stages[(size_t) i].name.c_str();
        if (ms) *ms = m->stage_totals[(size_t) i].ms_total;
        if (n_calls) *n_calls = m->stage_totals[(size_t) i].n_calls;
    });
}

}  // extern "C"
