// The .mcg parser and printer (reference: src/parser.cpp:26-436 for the
// language: line statements `graph`, `dim`, `input`, `const`, `output` and
// `name = op a, b`; `uniform(seed, lo, hi)` initialisers; dim overrides).

#include "minicompiler/parser.hpp"

#include "minicompiler/random.hpp"

#include <cctype>
#include <cerrno>
#include <cstdlib>
#include <fstream>
#include <sstream>
#include <unordered_map>
#include <vector>

namespace minicompiler {

namespace {

struct Token {
    enum class Kind { Word, Number, Symbol } kind;
    std::string text;
};

bool word_start(char c) { return std::isalpha(static_cast<unsigned char>(c)) || c == '_'; }
bool word_char(char c) { return std::isalnum(static_cast<unsigned char>(c)) || c == '_'; }
bool digit(char c) { return std::isdigit(static_cast<unsigned char>(c)) != 0; }

// One line into words, numbers (optionally signed, with exponent) and the
// symbols : = , [ ] ( ). `#` comments out the rest of the line.
Result<std::vector<Token>> lex_line(std::string_view line) {
    std::vector<Token> out;
    std::size_t i = 0;
    const std::size_t n = line.size();
    while (i < n) {
        const char c = line[i];
        if (std::isspace(static_cast<unsigned char>(c))) {
            ++i;
        } else if (c == '#') {
            break;
        } else if (word_start(c)) {
            std::size_t j = i;
            while (j < n && word_char(line[j])) ++j;
            out.push_back({Token::Kind::Word, std::string(line.substr(i, j - i))});
            i = j;
        } else if (digit(c) || c == '.' ||
                   ((c == '+' || c == '-') && i + 1 < n && (digit(line[i + 1]) || line[i + 1] == '.'))) {
            std::size_t j = i + 1;
            for (;;) {
                if (j < n && (digit(line[j]) || line[j] == '.')) {
                    ++j;
                } else if (j < n && (line[j] == 'e' || line[j] == 'E')) {
                    ++j;
                    if (j < n && (line[j] == '+' || line[j] == '-')) ++j;
                } else {
                    break;
                }
            }
            out.push_back({Token::Kind::Number, std::string(line.substr(i, j - i))});
            i = j;
        } else if (std::string_view(":=,[]()").find(c) != std::string_view::npos) {
            out.push_back({Token::Kind::Symbol, std::string(1, c)});
            ++i;
        } else {
            return Error{std::string("unexpected character '") + c + "'"};
        }
    }
    return out;
}

class Tokens {
public:
    explicit Tokens(std::vector<Token> t) : t_(std::move(t)) {}

    bool done() const { return at_ >= t_.size(); }
    bool is(Token::Kind k) const { return !done() && t_[at_].kind == k; }
    bool is_symbol(char c) const { return is(Token::Kind::Symbol) && t_[at_].text[0] == c; }
    const std::string& text() const { return t_[at_].text; }

    bool take_symbol(char c) {
        if (!is_symbol(c)) return false;
        ++at_;
        return true;
    }
    Status need_symbol(char c) {
        if (take_symbol(c)) return Status();
        return Error{std::string("expected '") + c + "' " + where()};
    }
    Result<std::string> word(const char* what) {
        if (!is(Token::Kind::Word)) return Error{std::string("expected ") + what + " " + where()};
        return t_[at_++].text;
    }
    Result<double> real(const char* what) {
        if (!is(Token::Kind::Number)) return Error{std::string("expected ") + what + " " + where()};
        const std::string& s = t_[at_++].text;
        char* end = nullptr;
        errno = 0;
        const double v = std::strtod(s.c_str(), &end);
        if (end != s.c_str() + s.size() || errno == ERANGE) return Error{"bad number '" + s + "'"};
        return v;
    }
    Result<std::int64_t> integer(const char* what) {
        if (!is(Token::Kind::Number)) return Error{std::string("expected ") + what + " " + where()};
        const std::string& s = t_[at_++].text;
        char* end = nullptr;
        errno = 0;
        const long long v = std::strtoll(s.c_str(), &end, 10);
        if (end != s.c_str() + s.size() || errno == ERANGE) return Error{"expected an integer, got '" + s + "'"};
        return static_cast<std::int64_t>(v);
    }
    std::string where() const { return done() ? "at end of line" : "but found '" + t_[at_].text + "'"; }

private:
    std::vector<Token> t_;
    std::size_t at_ = 0;
};

#define MC_TRY(expr)                       \
    do {                                   \
        Status mc_st_ = (expr);            \
        if (!mc_st_.ok()) return mc_st_;   \
    } while (0)

class Parser {
public:
    explicit Parser(const ParseOptions& options) : options_(options) {}

    Result<Graph> run(std::string_view text) {
        std::size_t line_no = 0;
        std::size_t pos = 0;
        for (;;) {
            std::size_t eol = text.find('\n', pos);
            const bool last = eol == std::string_view::npos;
            if (last) eol = text.size();
            std::string_view line = text.substr(pos, eol - pos);
            if (!line.empty() && line.back() == '\r') line.remove_suffix(1);
            ++line_no;
            Status st = line_statement(line);
            if (!st.ok()) return Error{"line " + std::to_string(line_no) + ": " + st.message()};
            if (last) break;
            pos = eol + 1;
        }
        for (const auto& kv : options_.dims) {
            if (dims_.count(kv.first) == 0) return Error{"the graph declares no dim '" + kv.first + "'"};
        }
        if (graph_.outputs().empty()) return Error{"the graph declares no outputs"};
        Status st = graph_.verify();
        if (!st.ok()) return st.error();
        return std::move(graph_);
    }

private:
    Status line_statement(std::string_view line) {
        Result<std::vector<Token>> lexed = lex_line(line);
        if (!lexed.ok()) return lexed.error();
        if (lexed->empty()) return Status();
        Tokens t(std::move(lexed).value());
        Result<std::string> head = t.word("a statement");
        if (!head.ok()) return head.error();
        const std::string& kw = head.value();
        if (kw == "graph") {
            MC_TRY(graph_statement(t));
        } else if (kw == "dim") {
            MC_TRY(dim_statement(t));
        } else if (kw == "input") {
            MC_TRY(input_statement(t));
        } else if (kw == "const") {
            MC_TRY(const_statement(t));
        } else if (kw == "output") {
            MC_TRY(output_statement(t));
        } else {
            MC_TRY(op_statement(t, kw));
        }
        if (!t.done()) return Error{"unexpected '" + t.text() + "'"};
        return Status();
    }

    Status graph_statement(Tokens& t) {
        Result<std::string> name = t.word("a graph name");
        if (!name.ok()) return name.error();
        if (graph_.num_nodes() != 0) return Error{"'graph' must come before any node"};
        graph_ = Graph(name.value());
        return Status();
    }

    Status dim_statement(Tokens& t) {
        Result<std::string> name = t.word("a dim name");
        if (!name.ok()) return name.error();
        MC_TRY(t.need_symbol('='));
        Result<std::int64_t> v = t.integer("a dim value");
        if (!v.ok()) return v.error();
        if (dims_.count(name.value())) return Error{"dim '" + name.value() + "' is declared twice"};
        const auto over = options_.dims.find(name.value());
        const std::int64_t value = over == options_.dims.end() ? v.value() : over->second;
        if (value < 1) return Error{"dim '" + name.value() + "' must be >= 1, got " + std::to_string(value)};
        dims_[name.value()] = value;
        return Status();
    }

    Status input_statement(Tokens& t) {
        Result<std::string> name = t.word("an input name");
        if (!name.ok()) return name.error();
        MC_TRY(t.need_symbol(':'));
        Result<TensorType> type = tensor_type(t);
        if (!type.ok()) return type.error();
        return bind(name.value(), graph_.add_input(name.value(), std::move(type).value()));
    }

    Status const_statement(Tokens& t) {
        Result<std::string> name = t.word("a constant name");
        if (!name.ok()) return name.error();
        MC_TRY(t.need_symbol(':'));
        Result<TensorType> type = tensor_type(t);
        if (!type.ok()) return type.error();
        MC_TRY(t.need_symbol('='));
        Result<std::vector<float>> values = initializer(t, type.value());
        if (!values.ok()) return values.error();
        return bind(name.value(), graph_.add_constant(name.value(), std::move(type).value(), std::move(values).value()));
    }

    Status output_statement(Tokens& t) {
        do {
            Result<std::string> name = t.word("an output name");
            if (!name.ok()) return name.error();
            Result<NodeId> id = lookup(name.value());
            if (!id.ok()) return id.error();
            MC_TRY(graph_.add_output(id.value()));
        } while (t.take_symbol(','));
        return Status();
    }

    Status op_statement(Tokens& t, const std::string& result_name) {
        if (!t.take_symbol('=')) return Error{"unknown statement '" + result_name + "'"};
        Result<std::string> word = t.word("an op name");
        if (!word.ok()) return word.error();
        const std::optional<OpKind> op = op_from_name(word.value());
        if (!op) return Error{"unknown op '" + word.value() + "'"};
        std::vector<NodeId> operands;
        do {
            Result<std::string> arg = t.word("an operand");
            if (!arg.ok()) return arg.error();
            Result<NodeId> id = lookup(arg.value());
            if (!id.ok()) return id.error();
            operands.push_back(id.value());
        } while (t.take_symbol(','));
        return bind(result_name, graph_.add_op(*op, std::move(operands), result_name));
    }

    Result<TensorType> tensor_type(Tokens& t) {
        Result<std::string> dtype = t.word("an element type");
        if (!dtype.ok()) return dtype.error();
        if (dtype.value() != "f32") return Error{"unsupported element type '" + dtype.value() + "' (only f32)"};
        Status st = t.need_symbol('[');
        if (!st.ok()) return st.error();
        Shape shape;
        if (!t.take_symbol(']')) {
            do {
                if (t.is(Token::Kind::Word)) {
                    const std::string dim = t.word("a dim").value();
                    const auto it = dims_.find(dim);
                    if (it == dims_.end()) return Error{"unknown dim '" + dim + "'"};
                    shape.push_back(it->second);
                } else {
                    Result<std::int64_t> d = t.integer("a dimension");
                    if (!d.ok()) return d.error();
                    shape.push_back(d.value());
                }
            } while (t.take_symbol(','));
            st = t.need_symbol(']');
            if (!st.ok()) return st.error();
        }
        // Before an initialiser allocates anything.
        if (!checked_num_elements(shape)) {
            return Error{"invalid shape " + to_string(shape) +
                         ": dimensions must be >= 1 and the total at most 2^31 - 1 elements"};
        }
        return TensorType(shape);
    }

    // `key=value` pairs of uniform(...) / normal(...).
    Result<std::map<std::string, std::string>> keyword_args(Tokens& t, const std::vector<std::string>& allowed,
                                                            const std::string& fn) {
        std::map<std::string, std::string> args;
        Status st = t.need_symbol('(');
        if (!st.ok()) return st.error();
        do {
            std::string names;
            for (const std::string& a : allowed) names += (names.empty() ? "" : ", ") + a;
            Result<std::string> key = t.word(names.c_str());
            if (!key.ok()) return key.error();
            bool known = false;
            for (const std::string& a : allowed) known = known || a == key.value();
            if (!known) return Error{fn + "() takes " + names + ", not '" + key.value() + "'"};
            st = t.need_symbol('=');
            if (!st.ok()) return st.error();
            if (!t.is(Token::Kind::Number)) return Error{"expected a number " + t.where()};
            args[key.value()] = t.text();
            if (key.value() == "seed") {
                Result<std::int64_t> s = t.integer("a seed");
                if (!s.ok()) return s.error();
                if (s.value() < 0) return Error{"seed must be >= 0"};
            } else {
                Result<double> v = t.real("a number");
                if (!v.ok()) return v.error();
            }
        } while (t.take_symbol(','));
        st = t.need_symbol(')');
        if (!st.ok()) return st.error();
        if (args.size() != allowed.size()) {
            std::string names;
            for (const std::string& a : allowed) names += (names.empty() ? "" : ", ") + a;
            return Error{fn + "() needs " + names};
        }
        return args;
    }

    Result<std::vector<float>> initializer(Tokens& t, const TensorType& type) {
        const std::size_t n = type.num_elements();
        if (t.is(Token::Kind::Number)) {
            const double v = t.real("a value").value();
            return std::vector<float>(n, static_cast<float>(v));
        }
        if (t.take_symbol('[')) {
            std::vector<float> values;
            do {
                Result<double> v = t.real("a value");
                if (!v.ok()) return v.error();
                values.push_back(static_cast<float>(v.value()));
            } while (t.take_symbol(','));
            Status st = t.need_symbol(']');
            if (!st.ok()) return st.error();
            if (values.size() != n) {
                return Error{"expected " + std::to_string(n) + " values for " + to_string(type) + ", got " +
                             std::to_string(values.size())};
            }
            return values;
        }
        Result<std::string> fn = t.word("a value, [values], uniform(...) or normal(...)");
        if (!fn.ok()) return fn.error();
        // Seeds stay integers: a double loses bits above 2^53.
        if (fn.value() == "uniform") {
            auto args = keyword_args(t, {"seed", "lo", "hi"}, "uniform");
            if (!args.ok()) return args.error();
            const auto seed = static_cast<std::uint64_t>(std::strtoll(args->at("seed").c_str(), nullptr, 10));
            const auto lo = static_cast<float>(std::strtod(args->at("lo").c_str(), nullptr));
            const auto hi = static_cast<float>(std::strtod(args->at("hi").c_str(), nullptr));
            if (!(lo < hi)) return Error{"uniform() needs lo < hi"};
            return uniform_values(n, seed, lo, hi);
        }
        if (fn.value() == "normal") {
            auto args = keyword_args(t, {"seed", "mean", "std"}, "normal");
            if (!args.ok()) return args.error();
            const auto seed = static_cast<std::uint64_t>(std::strtoll(args->at("seed").c_str(), nullptr, 10));
            const double mean = std::strtod(args->at("mean").c_str(), nullptr);
            const double sd = std::strtod(args->at("std").c_str(), nullptr);
            if (!(sd > 0.0)) return Error{"normal() needs std > 0"};
            return normal_values(n, seed, mean, sd);
        }
        return Error{"unknown initializer '" + fn.value() + "'"};
    }

    Result<NodeId> lookup(const std::string& name) const {
        const auto it = names_.find(name);
        if (it == names_.end()) return Error{"unknown value '" + name + "'"};
        return it->second;
    }

    Status bind(const std::string& name, Result<NodeId> id) {
        if (!id.ok()) return id.error();
        if (!names_.emplace(name, id.value()).second) return Error{"'" + name + "' is defined twice"};
        return Status();
    }

    const ParseOptions& options_;
    Graph graph_;
    std::map<std::string, std::int64_t> dims_;
    std::unordered_map<std::string, NodeId> names_;
};

#undef MC_TRY

}  // namespace

Result<Graph> parse_graph(std::string_view text, const ParseOptions& options) { return Parser(options).run(text); }

Result<Graph> parse_graph_file(const std::string& path, const ParseOptions& options) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return Error{"cannot open '" + path + "'"};
    std::stringstream buf;
    buf << f.rdbuf();
    Result<Graph> g = parse_graph(buf.str(), options);
    if (!g.ok()) return Error{path + ": " + g.error().message};
    return g;
}

std::string describe_constant(const Node& constant) {
    const std::vector<float>& v = *constant.constant;
    std::ostringstream os;
    if (v.size() == 1) {
        os << v[0];
    } else if (v.size() <= 4) {
        os << '[';
        for (std::size_t i = 0; i < v.size(); ++i) os << (i ? ", " : "") << v[i];
        os << ']';
    } else {
        os << '<' << v.size() << " values>";
    }
    return os.str();
}

std::string print_graph(const Graph& graph) {
    std::ostringstream os;
    os << "graph " << graph.name() << "\n";
    for (std::size_t i = 0; i < graph.num_nodes(); ++i) {
        const auto id = static_cast<NodeId>(i);
        const Node& n = graph.node(id);
        os << "  %" << id << ' ' << n.name << " = ";
        if (n.op == OpKind::Constant) {
            os << "const " << describe_constant(n);
        } else {
            os << op_name(n.op);
            for (std::size_t k = 0; k < n.inputs.size(); ++k) os << (k ? ", %" : " %") << n.inputs[k];
        }
        os << " : " << to_string(n.type);
        if (graph.is_output(id)) os << "  (output)";
        os << "\n";
        if (n.op == OpKind::FusedElementwise) {
            std::istringstream body(to_string(*n.fused));
            for (std::string line; std::getline(body, line);) os << "        " << line << "\n";
        }
    }
    return os.str();
}

}  // namespace minicompiler
