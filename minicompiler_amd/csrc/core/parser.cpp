// The .mcg reader and printer.
//
// The language is the reference's (include/minicompiler/parser.hpp:12-38,
// src/parser.cpp): one statement per line, `graph`, `dim`, `input`, `const`,
// `output` and `name = op a, b`, `#` comments, `uniform(seed, lo, hi)`
// initialisers and dim overrides; the messages the reference's tests compare
// (tests/test_parser.cpp:66-92) and the printer's line format
// (tests/test_parser.cpp:117-124) are kept word for word.
//
// The reader here is a lazy scanner over the whole text (statements end at a
// newline token, so no line is split off beforehand) feeding a reader whose
// steps are predicates: each returns false after recording the first
// failure, and a statement is a chain of `&&`. Statement keywords and
// initialisers are looked up in tables.

#include "minicompiler/parser.hpp"

#include "minicompiler/random.hpp"

#include <algorithm>
#include <array>
#include <charconv>
#include <cstdio>
#include <fstream>
#include <initializer_list>
#include <iterator>
#include <optional>
#include <unordered_map>
#include <vector>

namespace minicompiler {

namespace {

enum class Kind { Name, Number, Punct, Newline, Eof, Invalid };

struct Lexeme {
    Kind kind = Kind::Eof;
    std::string_view text;
    int line = 1;
};

bool is_alpha(char c) { return (c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z') || c == '_'; }
bool is_digit(char c) { return c >= '0' && c <= '9'; }

// Produces one lexeme at a time from the whole text. A number is an optional
// sign, a mantissa of digits with at most one '.', and an optional exponent
// (e or E, optional sign, digits). Punctuation is one of : = , [ ] ( ).
class Scanner {
public:
    explicit Scanner(std::string_view text) : src_(text) { advance(); }

    const Lexeme& peek() const { return cur_; }
    Lexeme take() {
        Lexeme out = cur_;
        advance();
        return out;
    }

private:
    char at(std::size_t i) const { return i < src_.size() ? src_[i] : '\0'; }

    std::size_t number_end(std::size_t i) const {
        if (at(i) == '+' || at(i) == '-') ++i;
        bool dot = false;
        for (; is_digit(at(i)) || (at(i) == '.' && !dot); ++i) {
            if (at(i) == '.') dot = true;
        }
        if (at(i) == 'e' || at(i) == 'E') {
            std::size_t j = i + 1;
            if (at(j) == '+' || at(j) == '-') ++j;
            if (is_digit(at(j))) {
                while (is_digit(at(j))) ++j;
                i = j;
            }
        }
        return i;
    }

    void advance() {
        for (;;) {
            const char c = at(pos_);
            if (c == ' ' || c == '\t' || c == '\r' || c == '\f' || c == '\v') {
                ++pos_;
            } else if (c == '#') {
                while (pos_ < src_.size() && src_[pos_] != '\n') ++pos_;
            } else {
                break;
            }
        }
        const std::size_t start = pos_;
        cur_.line = line_;
        if (pos_ >= src_.size()) {
            cur_.kind = Kind::Eof;
            cur_.text = {};
            return;
        }
        const char c = src_[pos_];
        std::size_t end = pos_ + 1;
        if (c == '\n') {
            cur_.kind = Kind::Newline;
            ++line_;
        } else if (is_alpha(c)) {
            while (is_alpha(at(end)) || is_digit(at(end))) ++end;
            cur_.kind = Kind::Name;
        } else if (is_digit(c) || c == '.' ||
                   ((c == '+' || c == '-') && (is_digit(at(pos_ + 1)) || at(pos_ + 1) == '.'))) {
            end = number_end(pos_);
            cur_.kind = Kind::Number;
        } else if (std::string_view(":=,[]()").find(c) != std::string_view::npos) {
            cur_.kind = Kind::Punct;
        } else {
            cur_.kind = Kind::Invalid;
        }
        cur_.text = src_.substr(start, end - start);
        pos_ = end;
    }

    std::string_view src_;
    std::size_t pos_ = 0;
    int line_ = 1;
    Lexeme cur_;
};

// Keyword arguments of an initialiser: name -> number text.
using Args = std::vector<std::pair<std::string_view, std::string_view>>;

class Reader {
public:
    Reader(std::string_view text, const ParseOptions& options) : scan_(text), options_(options) {}

    Result<Graph> read() {
        while (scan_.peek().kind != Kind::Eof) {
            if (scan_.peek().kind == Kind::Newline) {
                scan_.take();
                continue;
            }
            line_ = scan_.peek().line;
            if (!(statement() && statement_end())) return Error{"line " + std::to_string(line_) + ": " + failure_};
        }
        for (const auto& [name, value] : options_.dims) {
            (void)value;
            if (dims_.find(name) == dims_.end()) return Error{"the graph declares no dim '" + name + "'"};
        }
        if (graph_.outputs().empty()) return Error{"the graph declares no outputs"};
        if (Status st = graph_.verify(); !st.ok()) return st.error();
        return std::move(graph_);
    }

private:
    using Step = bool (Reader::*)();

    // -- failure and lexeme predicates
    bool fail(std::string message) {
        if (failure_.empty()) failure_ = std::move(message);
        return false;
    }
    bool invalid_here() {
        return fail(std::string("unexpected character '") + std::string(scan_.peek().text) + "'");
    }
    std::string found() const {
        const Lexeme& l = scan_.peek();
        if (l.kind == Kind::Newline || l.kind == Kind::Eof) return "before the end of the line";
        return "where '" + std::string(l.text) + "' stands";
    }
    bool expect(Kind kind, const char* what, std::string_view* text) {
        if (scan_.peek().kind == Kind::Invalid) return invalid_here();
        if (scan_.peek().kind != kind) return fail(std::string("expected ") + what + " " + found());
        *text = scan_.take().text;
        return true;
    }
    bool name(const char* what, std::string* out) {
        std::string_view t;
        if (!expect(Kind::Name, what, &t)) return false;
        out->assign(t);
        return true;
    }
    bool punct(char c) {
        std::string_view t;
        const char what[] = {'\'', c, '\'', '\0'};
        return expect(Kind::Punct, what, &t) && (t[0] == c || fail(std::string("expected ") + what + " where '" +
                                                                    std::string(t) + "' stands"));
    }
    bool maybe(char c) {
        if (scan_.peek().kind != Kind::Punct || scan_.peek().text[0] != c) return false;
        scan_.take();
        return true;
    }
    bool statement_end() {
        const Lexeme& l = scan_.peek();
        if (l.kind == Kind::Newline || l.kind == Kind::Eof) return true;
        if (l.kind == Kind::Invalid) return invalid_here();
        return fail("unexpected '" + std::string(l.text) + "'");
    }

    // -- numbers
    bool number_text(const char* what, std::string_view* text) { return expect(Kind::Number, what, text); }
    bool to_real(std::string_view t, double* out) {
        std::string_view s = !t.empty() && t[0] == '+' ? t.substr(1) : t;
        const auto r = std::from_chars(s.data(), s.data() + s.size(), *out);
        if (r.ec != std::errc() || r.ptr != s.data() + s.size()) {
            return fail("number '" + std::string(t) + "' is malformed or out of range");
        }
        return true;
    }
    bool to_integer(std::string_view t, std::int64_t* out) {
        std::string_view s = !t.empty() && t[0] == '+' ? t.substr(1) : t;
        const auto r = std::from_chars(s.data(), s.data() + s.size(), *out);
        if (r.ec != std::errc() || r.ptr != s.data() + s.size()) {
            return fail("'" + std::string(t) + "' is not a 64-bit integer");
        }
        return true;
    }
    bool real(const char* what, double* out) {
        std::string_view t;
        return number_text(what, &t) && to_real(t, out);
    }
    bool integer(const char* what, std::int64_t* out) {
        std::string_view t;
        return number_text(what, &t) && to_integer(t, out);
    }

    // -- names
    bool define(const std::string& label, Result<NodeId> id) {
        if (!id.ok()) return fail(id.error().message);
        if (!names_.emplace(label, id.value()).second) return fail("'" + label + "' is defined twice");
        return true;
    }
    bool value_named(const char* what, NodeId* out) {
        std::string label;
        if (!name(what, &label)) return false;
        const auto it = names_.find(label);
        if (it == names_.end()) return fail("unknown value '" + label + "'");
        *out = it->second;
        return true;
    }

    // -- statements
    bool statement() {
        static constexpr std::array<std::pair<std::string_view, Step>, 5> kKeywords = {{
            {"graph", &Reader::graph_line},
            {"dim", &Reader::dim_line},
            {"input", &Reader::input_line},
            {"const", &Reader::const_line},
            {"output", &Reader::output_line},
        }};
        std::string head;
        if (!name("a statement", &head)) return false;
        for (const auto& [word, step] : kKeywords) {
            if (word == head) return (this->*step)();
        }
        return assignment(head);
    }

    bool graph_line() {
        std::string label;
        if (!name("a graph name", &label)) return false;
        if (graph_.num_nodes() != 0) return fail("a 'graph' line has to precede every node");
        graph_ = Graph(label);
        return true;
    }

    bool dim_line() {
        std::string label;
        std::int64_t v = 0;
        if (!(name("a dim name", &label) && punct('=') && integer("the dim's size", &v))) return false;
        if (dims_.count(label)) return fail("dim '" + label + "' is already declared");
        if (const auto o = options_.dims.find(label); o != options_.dims.end()) v = o->second;
        if (v < 1) return fail("dim '" + label + "' = " + std::to_string(v) + " is not a positive size");
        dims_.emplace(label, v);
        return true;
    }

    bool input_line() {
        std::string label;
        TensorType type;
        return name("an input name", &label) && punct(':') && tensor_type(&type) &&
               define(label, graph_.add_input(label, type));
    }

    bool const_line() {
        std::string label;
        TensorType type;
        std::vector<float> values;
        return name("a constant name", &label) && punct(':') && tensor_type(&type) && punct('=') &&
               initializer(type, &values) && define(label, graph_.add_constant(label, type, std::move(values)));
    }

    bool output_line() {
        do {
            NodeId id = 0;
            if (!value_named("an output name", &id)) return false;
            if (Status st = graph_.add_output(id); !st.ok()) return fail(st.message());
        } while (maybe(','));
        return true;
    }

    bool assignment(const std::string& label) {
        if (!maybe('=')) return fail("'" + label + "' is neither a statement keyword nor an assignment");
        std::string op_word;
        if (!name("an op name", &op_word)) return false;
        const std::optional<OpKind> op = op_from_name(op_word);
        if (!op) return fail("unknown op '" + op_word + "'");
        std::vector<NodeId> operands;
        do {
            NodeId id = 0;
            if (!value_named("an operand", &id)) return false;
            operands.push_back(id);
        } while (maybe(','));
        return define(label, graph_.add_op(*op, std::move(operands), label));
    }

    // f32[d0, d1, ...]: each d a declared dim or an integer; checked before
    // any initialiser allocates.
    bool tensor_type(TensorType* out) {
        std::string dtype;
        if (!name("an element type", &dtype)) return false;
        if (dtype != "f32") return fail("unsupported element type '" + dtype + "' (only f32)");
        if (!punct('[')) return false;
        Shape shape;
        for (bool more = !maybe(']'); more; more = !maybe(']')) {
            if (!shape.empty() && !maybe(',')) return fail("expected ',' or ']' " + found());
            if (scan_.peek().kind == Kind::Name) {
                const std::string dim(scan_.take().text);
                const auto it = dims_.find(dim);
                if (it == dims_.end()) return fail("unknown dim '" + dim + "'");
                shape.push_back(it->second);
            } else {
                std::int64_t d = 0;
                if (!integer("a dimension", &d)) return false;
                shape.push_back(d);
            }
        }
        if (!checked_num_elements(shape)) {
            return fail("invalid shape " + to_string(shape) +
                        ": dimensions must be >= 1 and the total at most 2^31 - 1 elements");
        }
        *out = TensorType(shape);
        return true;
    }

    // ( key = number {, key = number} ), every key of `keys` exactly once.
    bool keyword_args(std::string_view fn, std::initializer_list<std::string_view> keys, Args* out) {
        if (!punct('(')) return false;
        do {
            std::string key;
            std::string_view text;
            if (!(name("an argument name", &key) && punct('=') && number_text("a number", &text))) return false;
            if (std::find(keys.begin(), keys.end(), key) == keys.end()) {
                return fail(std::string(fn) + "() has no argument '" + key + "'");
            }
            for (const auto& kv : *out) {
                if (kv.first == key) return fail(std::string(fn) + "() is given '" + key + "' twice");
            }
            out->emplace_back(*std::find(keys.begin(), keys.end(), key), text);
        } while (maybe(','));
        if (!punct(')')) return false;
        for (std::string_view k : keys) {
            bool given = false;
            for (const auto& kv : *out) given = given || kv.first == k;
            if (!given) return fail(std::string(fn) + "() is missing '" + std::string(k) + "'");
        }
        return true;
    }
    std::string_view arg(const Args& args, std::string_view key) const {
        for (const auto& kv : args) {
            if (kv.first == key) return kv.second;
        }
        return {};
    }
    // Seeds are read as unsigned 64-bit integers (a double would lose bits
    // above 2^53).
    bool seed_of(const Args& args, std::uint64_t* out) {
        const std::string_view t = arg(args, "seed");
        const auto r = std::from_chars(t.data(), t.data() + t.size(), *out);
        if (r.ec != std::errc() || r.ptr != t.data() + t.size()) {
            return fail("seed '" + std::string(t) + "' is not a non-negative 64-bit integer");
        }
        return true;
    }

    bool uniform_init(std::size_t n, std::vector<float>* out) {
        Args args;
        std::uint64_t seed = 0;
        double lo = 0, hi = 0;
        if (!(keyword_args("uniform", {"seed", "lo", "hi"}, &args) && seed_of(args, &seed) &&
              to_real(arg(args, "lo"), &lo) && to_real(arg(args, "hi"), &hi))) {
            return false;
        }
        if (!(static_cast<float>(lo) < static_cast<float>(hi))) return fail("uniform(): lo must be below hi");
        *out = uniform_values(n, seed, static_cast<float>(lo), static_cast<float>(hi));
        return true;
    }

    bool normal_init(std::size_t n, std::vector<float>* out) {
        Args args;
        std::uint64_t seed = 0;
        double mean = 0, sd = 0;
        if (!(keyword_args("normal", {"seed", "mean", "std"}, &args) && seed_of(args, &seed) &&
              to_real(arg(args, "mean"), &mean) && to_real(arg(args, "std"), &sd))) {
            return false;
        }
        if (!(sd > 0.0)) return fail("normal(): std must be positive");
        *out = normal_values(n, seed, mean, sd);
        return true;
    }

    // A number (every element), [v0, v1, ...] (exactly one per element) or a
    // generator call.
    bool initializer(const TensorType& type, std::vector<float>* out) {
        const std::size_t n = type.num_elements();
        const Lexeme& l = scan_.peek();
        if (l.kind == Kind::Number) {
            double v = 0;
            if (!real("a value", &v)) return false;
            out->assign(n, static_cast<float>(v));
            return true;
        }
        if (maybe('[')) {
            out->clear();
            for (bool more = !maybe(']'); more; more = !maybe(']')) {
                double v = 0;
                if (!out->empty() && !maybe(',')) return fail("expected ',' or ']' " + found());
                if (!real("a value", &v)) return false;
                out->push_back(static_cast<float>(v));
            }
            if (out->size() != n) {
                return fail("expected " + std::to_string(n) + " values for " + to_string(type) + ", got " +
                            std::to_string(out->size()));
            }
            return true;
        }
        using Init = bool (Reader::*)(std::size_t, std::vector<float>*);
        static constexpr std::array<std::pair<std::string_view, Init>, 2> kInits = {{
            {"uniform", &Reader::uniform_init},
            {"normal", &Reader::normal_init},
        }};
        std::string fn;
        if (!name("a value, a [list] or an initializer", &fn)) return false;
        for (const auto& [word, init] : kInits) {
            if (word == fn) return (this->*init)(n, out);
        }
        return fail("no initializer named '" + fn + "' (uniform or normal)");
    }

    Scanner scan_;
    const ParseOptions& options_;
    Graph graph_;
    std::map<std::string, std::int64_t> dims_;
    std::unordered_map<std::string, NodeId> names_;
    std::string failure_;
    int line_ = 1;
};

std::string format_float(float v) {
    char buf[32];
    std::snprintf(buf, sizeof buf, "%g", static_cast<double>(v));
    return buf;
}

}  // namespace

Result<Graph> parse_graph(std::string_view text, const ParseOptions& options) {
    return Reader(text, options).read();
}

Result<Graph> parse_graph_file(const std::string& path, const ParseOptions& options) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return Error{"cannot open '" + path + "'"};
    const std::string text((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    Result<Graph> g = parse_graph(text, options);
    if (!g.ok()) return Error{path + ": " + g.error().message};
    return g;
}

std::string describe_constant(const Node& constant) {
    const std::vector<float>& v = *constant.constant;
    if (v.size() == 1) return format_float(v[0]);
    if (v.size() > 4) return "<" + std::to_string(v.size()) + " values>";
    std::string s = "[";
    for (std::size_t i = 0; i < v.size(); ++i) s += (i ? ", " : "") + format_float(v[i]);
    return s + "]";
}

// Per node: "  %<id> <name> = <op> %a, %b : <type>[  (output)]", constants
// as "const <values>", fused groups followed by their program indented.
std::string print_graph(const Graph& graph) {
    std::string out = "graph " + graph.name() + "\n";
    for (NodeId id = 0; static_cast<std::size_t>(id) < graph.num_nodes(); ++id) {
        const Node& n = graph.node(id);
        std::string rhs;
        if (n.op == OpKind::Constant) {
            rhs = "const " + describe_constant(n);
        } else {
            rhs = op_name(n.op);
            const char* sep = " %";
            for (NodeId in : n.inputs) {
                rhs += sep + std::to_string(in);
                sep = ", %";
            }
        }
        out += "  %" + std::to_string(id) + " " + n.name + " = " + rhs + " : " + to_string(n.type) +
               (graph.is_output(id) ? "  (output)\n" : "\n");
        if (n.op == OpKind::FusedElementwise) {
            const std::string body = to_string(*n.fused);
            std::size_t at = 0;
            while (at < body.size()) {
                std::size_t eol = body.find('\n', at);
                if (eol == std::string::npos) eol = body.size();
                out += "        " + body.substr(at, eol - at) + "\n";
                at = eol + 1;
            }
        }
    }
    return out;
}

}  // namespace minicompiler
