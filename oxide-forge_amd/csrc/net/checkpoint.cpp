// checkpoint.cpp -- checkpoint format version 1 (include/oxforge_checkpoint.hpp).
//
// The metadata file is TOML.  Only the subset the format uses is read:
// comments, `key = value` with integer, string or boolean values (and
// inline tables of those), `[table.path]` headers and `[[array.path]]`
// arrays of tables -- what any TOML serializer emits for these structures.
// Files are written in the layout of a pretty-printed TOML document (plain
// keys first, then one header per nested table).
#include "oxforge_checkpoint.hpp"

#include <cctype>
#include <cerrno>
#include <climits>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <sstream>

namespace oxforge {
namespace checkpoint {
namespace {

static_assert(sizeof(float) == 4, "f32 parameters");

[[noreturn]] void invalid(const std::string& msg) { throw Error(FORGE_EINVAL, "checkpoint: " + msg); }
[[noreturn]] void io_error(const std::string& msg) {
    throw Error(FORGE_EIO, "checkpoint: " + msg + ": " + std::strerror(errno));
}

// ------------------------------------------------------------ TOML subset

struct Value {
    enum Kind { Int, Str, Bool } kind = Int;
    long long i = 0;
    std::string s;
    bool b = false;
};

struct Table {
    std::map<std::string, Value> values;
    std::map<std::string, std::unique_ptr<Table>> tables;
    std::map<std::string, std::vector<std::unique_ptr<Table>>> arrays;
    // How the table came to exist.  TOML 1.0 allows a table to be defined
    // once: by its [header], by dotted keys, or as an inline table; a table
    // created only as the parent of another header may get its own header
    // later.
    bool by_header = false, by_dotted_key = false, is_inline = false;

    bool has_key(const std::string& k) const {
        return values.count(k) || tables.count(k) || arrays.count(k);
    }
};

class Parser {
public:
    explicit Parser(const std::string& text) : text_(text) {}

    std::unique_ptr<Table> parse() {
        auto root = std::make_unique<Table>();
        Table* cur = root.get();
        std::istringstream in(text_);
        std::string raw;
        while (std::getline(in, raw)) {
            line_++;
            std::string l = trim(strip_comment(raw));
            if (l.empty()) continue;
            if (l.rfind("[[", 0) == 0) {
                if (l.size() < 4 || l.compare(l.size() - 2, 2, "]]") != 0) fail("bad array header");
                auto path = split_key(l.substr(2, l.size() - 4));
                Table* parent = root.get();
                for (size_t i = 0; i + 1 < path.size(); i++) parent = child(parent, path[i]);
                const std::string& last = path.back();
                if (parent->values.count(last) || parent->tables.count(last))
                    fail("key '" + last + "' is not an array of tables");
                parent->arrays[last].push_back(std::make_unique<Table>());
                cur = parent->arrays[last].back().get();
            } else if (l[0] == '[') {
                if (l.back() != ']') fail("bad table header");
                auto path = split_key(l.substr(1, l.size() - 2));
                Table* t = root.get();
                for (const auto& seg : path) t = child(t, seg);
                if (t->by_header || t->by_dotted_key || t->is_inline)
                    fail("table '" + join(path) + "' defined twice");
                t->by_header = true;
                cur = t;
            } else {
                size_t eq = find_unquoted(l, '=');
                if (eq == std::string::npos) fail("expected key = value");
                auto path = split_key(l.substr(0, eq));
                Table* t = cur;
                for (size_t i = 0; i + 1 < path.size(); i++) {
                    t = child(t, path[i]);
                    if (t->by_header) fail("table '" + path[i] + "' defined twice");
                    t->by_dotted_key = true;
                }
                size_t pos = 0;
                std::string rest = trim(l.substr(eq + 1));
                assign(t, path.back(), rest, pos);
                if (!trim(rest.substr(pos)).empty()) fail("trailing characters after value");
            }
        }
        return root;
    }

private:
    [[noreturn]] void fail(const std::string& msg) const {
        invalid("TOML line " + std::to_string(line_) + ": " + msg);
    }

    static std::string trim(const std::string& s) {
        size_t a = s.find_first_not_of(" \t\r");
        if (a == std::string::npos) return "";
        size_t b = s.find_last_not_of(" \t\r");
        return s.substr(a, b - a + 1);
    }

    static std::string strip_comment(const std::string& s) {
        char quote = 0;
        for (size_t i = 0; i < s.size(); i++) {
            char c = s[i];
            if (quote) {
                if (c == '\\' && quote == '"') i++;
                else if (c == quote) quote = 0;
            } else if (c == '"' || c == '\'') {
                quote = c;
            } else if (c == '#') {
                return s.substr(0, i);
            }
        }
        return s;
    }

    static size_t find_unquoted(const std::string& s, char target) {
        char quote = 0;
        for (size_t i = 0; i < s.size(); i++) {
            char c = s[i];
            if (quote) {
                if (c == '\\' && quote == '"') i++;
                else if (c == quote) quote = 0;
            } else if (c == '"' || c == '\'') {
                quote = c;
            } else if (c == target) {
                return i;
            }
        }
        return std::string::npos;
    }

    std::vector<std::string> split_key(const std::string& key) const {
        std::vector<std::string> out;
        std::string k = trim(key);
        size_t i = 0;
        while (i <= k.size()) {
            while (i < k.size() && (k[i] == ' ' || k[i] == '\t')) i++;
            std::string seg;
            if (i < k.size() && (k[i] == '"' || k[i] == '\'')) {
                char q = k[i++];
                while (i < k.size() && k[i] != q) seg += k[i++];
                if (i >= k.size()) fail("unterminated quoted key");
                i++;
            } else {
                while (i < k.size() && k[i] != '.' && k[i] != ' ' && k[i] != '\t') {
                    char c = k[i];
                    if (!(isalnum((unsigned char)c) || c == '_' || c == '-')) fail("bad key character");
                    seg += c;
                    i++;
                }
                if (seg.empty()) fail("empty key");
            }
            out.push_back(seg);
            while (i < k.size() && (k[i] == ' ' || k[i] == '\t')) i++;
            if (i >= k.size()) break;
            if (k[i] != '.') fail("bad dotted key");
            i++;
        }
        if (out.empty()) fail("empty key");
        return out;
    }

    static std::string join(const std::vector<std::string>& path) {
        std::string out;
        for (const auto& seg : path) out += (out.empty() ? "" : ".") + seg;
        return out;
    }

    // The sub-table `name` of t: an existing table, the last element of an
    // array of tables, or a new table.  Inline tables are closed.
    Table* child(Table* t, const std::string& name) const {
        auto it = t->tables.find(name);
        if (it != t->tables.end()) {
            if (it->second->is_inline) fail("inline table '" + name + "' cannot be extended");
            return it->second.get();
        }
        auto at = t->arrays.find(name);
        if (at != t->arrays.end()) {
            if (at->second.empty()) fail("empty array of tables");
            return at->second.back().get();
        }
        if (t->values.count(name)) fail("key '" + name + "' is not a table");
        auto& slot = t->tables[name];
        slot = std::make_unique<Table>();
        return slot.get();
    }

    void assign(Table* t, const std::string& key, const std::string& s, size_t& pos) const {
        if (t->has_key(key)) fail("duplicate key '" + key + "'");
        if (pos < s.size() && s[pos] == '{') {
            auto& slot = t->tables[key];
            slot = std::make_unique<Table>();
            slot->is_inline = true;
            pos++;
            skip_ws(s, pos);
            if (pos < s.size() && s[pos] == '}') {
                pos++;
                return;
            }
            while (true) {
                skip_ws(s, pos);
                size_t eq = s.find('=', pos);
                if (eq == std::string::npos) fail("bad inline table");
                auto path = split_key(s.substr(pos, eq - pos));
                if (path.size() != 1) fail("dotted key in inline table");
                pos = eq + 1;
                skip_ws(s, pos);
                assign(slot.get(), path[0], s, pos);
                skip_ws(s, pos);
                if (pos < s.size() && s[pos] == ',') {
                    pos++;
                    continue;
                }
                if (pos < s.size() && s[pos] == '}') {
                    pos++;
                    return;
                }
                fail("bad inline table");
            }
        }
        t->values[key] = parse_scalar(s, pos);
    }

    static void skip_ws(const std::string& s, size_t& pos) {
        while (pos < s.size() && (s[pos] == ' ' || s[pos] == '\t')) pos++;
    }

    Value parse_scalar(const std::string& s, size_t& pos) const {
        Value v;
        if (pos >= s.size()) fail("missing value");
        char c = s[pos];
        if (c == '"' || c == '\'') {
            v.kind = Value::Str;
            pos++;
            while (pos < s.size() && s[pos] != c) {
                if (c == '"' && s[pos] == '\\') {
                    if (++pos >= s.size()) fail("bad escape");
                    switch (s[pos]) {
                    case '"': v.s += '"'; break;
                    case '\\': v.s += '\\'; break;
                    case 'n': v.s += '\n'; break;
                    case 't': v.s += '\t'; break;
                    case 'r': v.s += '\r'; break;
                    default: fail("unsupported escape");
                    }
                    pos++;
                } else {
                    v.s += s[pos++];
                }
            }
            if (pos >= s.size()) fail("unterminated string");
            pos++;
            return v;
        }
        if (s.compare(pos, 4, "true") == 0) {
            v.kind = Value::Bool;
            v.b = true;
            pos += 4;
            return v;
        }
        if (s.compare(pos, 5, "false") == 0) {
            v.kind = Value::Bool;
            pos += 5;
            return v;
        }
        v.kind = Value::Int;
        bool neg = false;
        if (c == '+' || c == '-') {
            neg = c == '-';
            pos++;
        }
        size_t start = pos;
        unsigned long long acc = 0;
        while (pos < s.size() && (isdigit((unsigned char)s[pos]) || s[pos] == '_')) {
            if (s[pos] != '_') {
                unsigned long long d = (unsigned long long)(s[pos] - '0');
                if (acc > (~0ull - d) / 10) fail("integer overflow");
                acc = acc * 10 + d;
            } else if (pos == start || pos + 1 >= s.size() || !isdigit((unsigned char)s[pos - 1]) ||
                       !isdigit((unsigned char)s[pos + 1])) {
                // TOML: each underscore between two digits.
                fail("misplaced underscore in integer");
            }
            pos++;
        }
        if (pos == start) fail("unsupported value (only integers, strings and booleans)");
        if (s[start] == '0' && pos - start > 1) fail("leading zeros are not allowed in integers");
        if (pos < s.size() && (s[pos] == '.' || s[pos] == 'e' || s[pos] == 'E'))
            fail("floating-point values are not part of the format");
        if (acc > (unsigned long long)LLONG_MAX) fail("integer overflow");
        v.i = neg ? -(long long)acc : (long long)acc;
        return v;
    }

    const std::string& text_;
    size_t line_ = 0;
};

// Typed access with the reference's error wording.
const Value& need_value(const Table& t, const std::string& key, const std::string& where) {
    auto it = t.values.find(key);
    if (it == t.values.end()) invalid(where + ": missing field '" + key + "'");
    return it->second;
}
uint64_t need_u64(const Table& t, const std::string& key, const std::string& where) {
    const Value& v = need_value(t, key, where);
    if (v.kind != Value::Int || v.i < 0) invalid(where + ": '" + key + "' must be a non-negative integer");
    return (uint64_t)v.i;
}
std::string need_str(const Table& t, const std::string& key, const std::string& where) {
    const Value& v = need_value(t, key, where);
    if (v.kind != Value::Str) invalid(where + ": '" + key + "' must be a string");
    return v.s;
}
bool need_bool(const Table& t, const std::string& key, const std::string& where) {
    const Value& v = need_value(t, key, where);
    if (v.kind != Value::Bool) invalid(where + ": '" + key + "' must be a boolean");
    return v.b;
}
const Table* opt_table(const Table& t, const std::string& key) {
    auto it = t.tables.find(key);
    return it == t.tables.end() ? nullptr : it->second.get();
}
const Table& need_table(const Table& t, const std::string& key, const std::string& where) {
    const Table* s = opt_table(t, key);
    if (!s) invalid(where + ": missing table '" + key + "'");
    return *s;
}

// ------------------------------------------------- metadata <-> TOML

const char* activation_name(Activation a) {
    switch (a) {
    case Activation::Identity: return "identity";
    case Activation::Gelu: return "gelu";
    case Activation::Relu: return "relu";
    case Activation::Silu: return "silu";
    }
    return "identity";
}
Activation parse_activation(const std::string& s) {
    if (s == "identity") return Activation::Identity;
    if (s == "gelu") return Activation::Gelu;
    if (s == "relu") return Activation::Relu;
    if (s == "silu") return Activation::Silu;
    invalid("unknown activation \"" + s + "\"");
}
const char* norm_name(NormType n) { return n == NormType::Rms ? "rms" : "layer"; }
NormType parse_norm(const std::string& s) {
    if (s == "rms") return NormType::Rms;
    if (s == "layer") return NormType::Layer;
    invalid("unknown normalization \"" + s + "\"");
}

MatrixMetadata read_matrix(const Table& t, const std::string& where) {
    MatrixMetadata m;
    m.rows = need_u64(t, "rows", where);
    m.cols = need_u64(t, "cols", where);
    m.byte_start = need_u64(t, "byte_start", where);
    m.byte_end = need_u64(t, "byte_end", where);
    return m;
}
VectorMetadata read_vector(const Table& t, const std::string& where) {
    VectorMetadata v;
    v.len = need_u64(t, "len", where);
    v.byte_start = need_u64(t, "byte_start", where);
    v.byte_end = need_u64(t, "byte_end", where);
    return v;
}
LinearMetadata read_linear(const Table& t, const std::string& where) {
    LinearMetadata l;
    l.input_neurons = need_u64(t, "input_neurons", where);
    l.output_neurons = need_u64(t, "output_neurons", where);
    l.activation = parse_activation(need_str(t, "activation", where));
    l.weights = read_matrix(need_table(t, "weights", where), where + ".weights");
    if (const Table* b = opt_table(t, "bias")) l.bias = read_vector(*b, where + ".bias");
    return l;
}
MlpMetadata read_mlp(const Table& t, const std::string& where) {
    MlpMetadata m;
    m.layer_count = need_u64(t, "layer_count", where);
    const std::string loss = need_str(t, "loss", where);
    if (loss != "mean_squared_error") invalid(where + ": unknown loss \"" + loss + "\"");
    if (const Table* r = opt_table(t, "residual")) {
        m.residual = ResidualMetadata{need_u64(*r, "start", where + ".residual"),
                                      need_u64(*r, "end", where + ".residual")};
    }
    auto it = t.arrays.find("layers");
    if (it != t.arrays.end()) {
        for (size_t i = 0; i < it->second.size(); i++)
            m.layers.push_back(read_linear(*it->second[i], where + ".layers[" + std::to_string(i) + "]"));
    }
    return m;
}
TransformerMetadata read_transformer(const Table& t, const std::string& where) {
    TransformerMetadata m;
    m.block_count = need_u64(t, "block_count", where);
    m.attention_residual = need_bool(t, "attention_residual", where);
    m.feed_forward_residual = need_bool(t, "feed_forward_residual", where);
    m.normalization = parse_norm(need_str(t, "normalization", where));
    m.position = read_matrix(need_table(t, "position", where), where + ".position");
    m.query = read_linear(need_table(t, "query", where), where + ".query");
    m.key = read_linear(need_table(t, "key", where), where + ".key");
    m.value = read_linear(need_table(t, "value", where), where + ".value");
    m.feed_forward = read_mlp(need_table(t, "feed_forward", where), where + ".feed_forward");
    m.output = read_linear(need_table(t, "output", where), where + ".output");
    const char* ext[4] = {"norm1_gamma", "norm1_beta", "norm2_gamma", "norm2_beta"};
    std::optional<VectorMetadata>* dst[4] = {&m.norm1_gamma, &m.norm1_beta, &m.norm2_gamma,
                                             &m.norm2_beta};
    for (int i = 0; i < 4; i++)
        if (const Table* v = opt_table(t, ext[i])) *dst[i] = read_vector(*v, where + "." + ext[i]);
    return m;
}

void write_matrix(std::ostream& o, const std::string& path, const MatrixMetadata& m) {
    o << "\n[" << path << "]\nrows = " << m.rows << "\ncols = " << m.cols
      << "\nbyte_start = " << m.byte_start << "\nbyte_end = " << m.byte_end << "\n";
}
void write_vector(std::ostream& o, const std::string& path, const VectorMetadata& v) {
    o << "\n[" << path << "]\nlen = " << v.len << "\nbyte_start = " << v.byte_start
      << "\nbyte_end = " << v.byte_end << "\n";
}
void write_linear_body(std::ostream& o, const std::string& path, const LinearMetadata& l) {
    o << "input_neurons = " << l.input_neurons << "\noutput_neurons = " << l.output_neurons
      << "\nactivation = \"" << activation_name(l.activation) << "\"\n";
    write_matrix(o, path + ".weights", l.weights);
    if (l.bias) write_vector(o, path + ".bias", *l.bias);
}
void write_linear(std::ostream& o, const std::string& path, const LinearMetadata& l) {
    o << "\n[" << path << "]\n";
    write_linear_body(o, path, l);
}
void write_mlp(std::ostream& o, const std::string& path, const MlpMetadata& m) {
    o << "\n[" << path << "]\nlayer_count = " << m.layer_count
      << "\nloss = \"mean_squared_error\"\n";
    if (m.residual)
        o << "\n[" << path << ".residual]\nstart = " << m.residual->start
          << "\nend = " << m.residual->end << "\n";
    for (const auto& l : m.layers) {
        o << "\n[[" << path << ".layers]]\n";
        write_linear_body(o, path + ".layers", l);
    }
}
void write_header(std::ostream& o, const char* model_type, const std::string& data_file,
                  uint64_t data_bytes) {
    o << "format_version = " << FORMAT_VERSION << "\nmodel_type = \"" << model_type
      << "\"\nscalar_type = \"f32_le\"\ndata_file = \"" << data_file
      << "\"\ndata_bytes = " << data_bytes << "\n";
}

// ------------------------------------------------------------ validation

// model.rs:494-536: ranges must follow each other from byte 0.
struct RangeValidator {
    uint64_t position = 0;
    void range(uint64_t start, uint64_t end, uint64_t elements) {
        if (elements > UINT64_MAX / 4) invalid("parameter byte length overflow");
        const uint64_t expected_end = position + elements * 4;
        if (expected_end < position) invalid("checkpoint offset overflow");
        if (start != position || end != expected_end)
            invalid("parameter range [" + std::to_string(start) + ", " + std::to_string(end) +
                    ") is not the expected contiguous range [" + std::to_string(position) +
                    ", " + std::to_string(expected_end) + ")");
        position = expected_end;
    }
    void matrix(const MatrixMetadata& m) {
        if (m.cols != 0 && m.rows > UINT64_MAX / m.cols) invalid("matrix element count overflow");
        range(m.byte_start, m.byte_end, (uint64_t)m.rows * m.cols);
    }
    void vector(const VectorMetadata& v) { range(v.byte_start, v.byte_end, v.len); }
    void finish(uint64_t data_bytes) const {
        if (position != data_bytes)
            invalid("parameter ranges end at " + std::to_string(position) +
                    ", metadata declares " + std::to_string(data_bytes) + " bytes");
    }
};

void validate_linear(const LinearMetadata& l, RangeValidator& r) {
    // model.rs:400-417.
    if (l.input_neurons == 0 || l.output_neurons == 0) invalid("Linear dimensions must be non-zero");
    if (l.weights.rows != l.input_neurons || l.weights.cols != l.output_neurons)
        invalid("Linear weight shape does not match its neuron counts");
    r.matrix(l.weights);
    if (l.bias) {
        if (l.bias->len != l.output_neurons) invalid("Linear bias length does not match output neurons");
        r.vector(*l.bias);
    }
}

void validate_mlp(const MlpMetadata& m, RangeValidator& r) {
    // model.rs:366-398.
    if (m.layer_count == 0 || m.layer_count != m.layers.size())
        invalid("MLP layer_count is " + std::to_string(m.layer_count) + ", but " +
                std::to_string(m.layers.size()) + " layers are described");
    for (size_t i = 0; i < m.layers.size(); i++) {
        validate_linear(m.layers[i], r);
        if (i > 0 && m.layers[i - 1].output_neurons != m.layers[i].input_neurons)
            invalid("MLP layer " + std::to_string(i) + " expects " +
                    std::to_string(m.layers[i].input_neurons) + " neurons, previous layer produces " +
                    std::to_string(m.layers[i - 1].output_neurons));
    }
    if (m.residual) {
        if (m.residual->start >= m.residual->end || m.residual->end > m.layers.size())
            invalid("invalid MLP residual range");
        const size_t in = m.layers[m.residual->start].input_neurons;
        const size_t out = m.layers[m.residual->end - 1].output_neurons;
        if (in != out)
            invalid("residual connects " + std::to_string(in) + " input neurons to " +
                    std::to_string(out) + " output neurons");
    }
}

void validate_transformer(const TransformerMetadata& m, RangeValidator& r) {
    // model.rs:419-466, then the gamma/beta extension.
    if (m.block_count != 1) invalid("this Transformer executor requires exactly one block");
    if (!m.attention_residual || !m.feed_forward_residual)
        invalid("this Transformer executor requires both residual paths");
    validate_linear(m.query, r);
    validate_linear(m.key, r);
    validate_linear(m.value, r);
    r.matrix(m.position);
    validate_mlp(m.feed_forward, r);
    validate_linear(m.output, r);
    const size_t emb = m.position.cols;
    if (m.position.rows == 0 || emb == 0) invalid("position matrix dimensions must be non-zero");
    if (m.query.input_neurons != emb || m.key.input_neurons != emb || m.value.input_neurons != emb)
        invalid("Q/K/V input dimensions must match the embedding size");
    if (m.query.output_neurons != m.key.output_neurons) invalid("query and key dimensions must match");
    if (m.value.output_neurons != emb) invalid("value output dimension must match the residual embedding");
    if (m.feed_forward.layers.front().input_neurons != emb ||
        m.feed_forward.layers.back().output_neurons != emb)
        invalid("feed-forward input/output must match the embedding size");
    if (m.output.input_neurons != emb) invalid("output projection input must match the embedding size");
    const std::optional<VectorMetadata>* ext[4] = {&m.norm1_gamma, &m.norm1_beta, &m.norm2_gamma,
                                                   &m.norm2_beta};
    for (int i = 0; i < 4; i++) {
        if (!*ext[i]) continue;
        if ((*ext[i])->len != emb) invalid("norm gamma/beta length must match the embedding size");
        if ((i == 1 || i == 3) && m.normalization != NormType::Layer)
            invalid("norm beta is only defined for LayerNorm");
        r.vector(**ext[i]);
    }
}

void validate_header(const Table& root, const char* expected_type) {
    // model.rs:326-351.
    const uint64_t version = need_u64(root, "format_version", "checkpoint");
    if (version != FORMAT_VERSION)
        invalid("unsupported checkpoint format version " + std::to_string(version) +
                "; expected " + std::to_string(FORMAT_VERSION));
    const std::string type = need_str(root, "model_type", "checkpoint");
    if (type != expected_type)
        invalid("checkpoint contains model type \"" + type + "\", expected \"" + expected_type + "\"");
    const std::string scalar = need_str(root, "scalar_type", "checkpoint");
    if (scalar != "f32_le")
        invalid("unsupported scalar encoding \"" + scalar + "\"; expected \"f32_le\"");
}

// --------------------------------------------------------------- paths

// io.rs:20-29: no extension -> .toml; .toml kept; anything else rejected.
std::string metadata_path(const std::string& path) {
    const size_t slash = path.find_last_of('/');
    const std::string name = slash == std::string::npos ? path : path.substr(slash + 1);
    const size_t dot = name.find_last_of('.');
    if (name.empty()) invalid("checkpoint path has no file name");
    if (dot == std::string::npos || dot == 0) return path + ".toml";
    const std::string ext = name.substr(dot + 1);
    if (ext == "toml") return path;
    invalid("checkpoint metadata must use .toml, not ." + ext);
}

std::string with_extension(const std::string& path, const std::string& ext) {
    const size_t slash = path.find_last_of('/');
    const size_t dot = path.find_last_of('.');
    if (dot != std::string::npos && (slash == std::string::npos || dot > slash + 1))
        return path.substr(0, dot) + "." + ext;
    return path + "." + ext;
}

std::string file_name(const std::string& path) {
    const size_t slash = path.find_last_of('/');
    return slash == std::string::npos ? path : path.substr(slash + 1);
}

// io.rs:38-50: data_file must be a plain file name next to the metadata.
std::string resolve_data_path(const std::string& meta, const std::string& data_file) {
    if (data_file.empty() || data_file == "." || data_file == ".." ||
        data_file.find('/') != std::string::npos)
        invalid("checkpoint data_file must be a plain file name");
    const size_t slash = meta.find_last_of('/');
    return slash == std::string::npos ? data_file : meta.substr(0, slash + 1) + data_file;
}

std::string read_text(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) io_error("cannot open " + path);
    std::ostringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

void write_text(const std::string& path, const std::string& text) {
    std::ofstream f(path, std::ios::binary | std::ios::trunc);
    if (!f) io_error("cannot create " + path);
    f << text;
    f.flush();
    if (!f) io_error("cannot write " + path);
}

// ------------------------------------------------------------- parameters

// Host copies of the parameters, in checkpoint order (the models' get_data).
struct Parameters {
    std::vector<HostData> blocks;
};

void write_parameters(const std::string& path, const Parameters& params, uint64_t expected) {
    // io.rs:66-123: contiguous little-endian f32 (the host is little-endian).
    std::ofstream f(path, std::ios::binary | std::ios::trunc);
    if (!f) io_error("cannot create " + path);
    uint64_t written = 0;
    for (const HostData& b : params.blocks) {
        const std::vector<float>& v = b.values();
        f.write(reinterpret_cast<const char*>(v.data()), (std::streamsize)(v.size() * 4));
        written += (uint64_t)v.size() * 4;
    }
    f.flush();
    if (!f) io_error("cannot write " + path);
    if (written != expected)
        invalid("model exported " + std::to_string(written) +
                " parameter bytes, metadata declares " + std::to_string(expected));
}

class ParameterReader {
public:
    ParameterReader(const std::string& path, uint64_t expected) : f_(path, std::ios::binary) {
        // io.rs:125-177.
        if (!f_) io_error("cannot open " + path);
        f_.seekg(0, std::ios::end);
        len_ = (uint64_t)f_.tellg();
        if (len_ != expected)
            invalid("data file has " + std::to_string(len_) + " bytes, metadata declares " +
                    std::to_string(expected));
    }
    std::vector<float> read(uint64_t start, uint64_t end, uint64_t values) {
        if (start > end || end > len_)
            invalid("parameter range [" + std::to_string(start) + ", " + std::to_string(end) +
                    ") is outside a " + std::to_string(len_) + " byte data file");
        if (end - start != values * 4)
            invalid("parameter range has " + std::to_string(end - start) + " bytes, expected " +
                    std::to_string(values * 4));
        std::vector<float> out(values);
        f_.seekg((std::streamoff)start);
        f_.read(reinterpret_cast<char*>(out.data()), (std::streamsize)(values * 4));
        if (!f_) io_error("cannot read parameters");
        return out;
    }

private:
    std::ifstream f_;
    uint64_t len_ = 0;
};

// ------------------------------------------------ model <-> metadata

Linear load_linear_params(const LinearMetadata& m, ParameterReader& r, CudaRuntime& rt) {
    std::vector<float> w = r.read(m.weights.byte_start, m.weights.byte_end,
                                  (uint64_t)m.weights.rows * m.weights.cols);
    Matrix W = rt.matrix_from_host(w, m.weights.rows, m.weights.cols);
    std::optional<Vector> b;
    if (m.bias) b = rt.vector_from_host(r.read(m.bias->byte_start, m.bias->byte_end, m.bias->len));
    return Linear(std::move(W), std::move(b), m.activation);
}

std::pair<std::vector<Linear>, std::optional<std::pair<size_t, size_t>>> load_mlp_params(
    const MlpMetadata& m, ParameterReader& r, CudaRuntime& rt) {
    std::vector<Linear> layers;
    for (const auto& l : m.layers) layers.push_back(load_linear_params(l, r, rt));
    std::optional<std::pair<size_t, size_t>> res;
    if (m.residual) res = std::make_pair(m.residual->start, m.residual->end);
    return {std::move(layers), res};
}

std::optional<Normalization> load_norm(NormType kind, const std::optional<VectorMetadata>& g,
                                       const std::optional<VectorMetadata>& b,
                                       ParameterReader& r, CudaRuntime& rt) {
    if (!g && !b) return std::nullopt;
    Normalization n;
    n.kind = kind;
    if (g) n.gamma = rt.vector_from_host(r.read(g->byte_start, g->byte_end, g->len));
    if (b) n.beta = rt.vector_from_host(r.read(b->byte_start, b->byte_end, b->len));
    return n;
}

// ------------------------------------------------------------ file level

struct Opened {
    std::string meta_path;
    std::unique_ptr<Table> root;
    uint64_t data_bytes = 0;
    std::string data_path;
};

Opened open_file(const std::string& path, const char* model_type) {
    Opened o;
    o.meta_path = metadata_path(path);
    o.root = Parser(read_text(o.meta_path)).parse();
    validate_header(*o.root, model_type);
    o.data_bytes = need_u64(*o.root, "data_bytes", "checkpoint");
    o.data_path = resolve_data_path(o.meta_path, need_str(*o.root, "data_file", "checkpoint"));
    return o;
}

void dump(const std::string& path, const char* model_type, const std::string& body,
          uint64_t data_bytes, const Parameters& params) {
    const std::string meta = metadata_path(path);
    const std::string data = with_extension(meta, "bin");
    std::ostringstream o;
    write_header(o, model_type, file_name(data), data_bytes);
    o << body;
    write_text(meta, o.str());
    write_parameters(data, params, data_bytes);
}

std::string linear_body(const LinearMetadata& m) {
    std::ostringstream o;
    write_linear(o, "linear", m);
    return o.str();
}
std::string mlp_body(const MlpMetadata& m) {
    std::ostringstream o;
    write_mlp(o, "mlp", m);
    return o.str();
}
std::string transformer_body(const TransformerMetadata& m) {
    std::ostringstream o;
    o << "\n[transformer]\nblock_count = " << m.block_count << "\nattention_residual = "
      << (m.attention_residual ? "true" : "false") << "\nfeed_forward_residual = "
      << (m.feed_forward_residual ? "true" : "false") << "\nnormalization = \""
      << norm_name(m.normalization) << "\"\n";
    write_matrix(o, "transformer.position", m.position);
    write_linear(o, "transformer.query", m.query);
    write_linear(o, "transformer.key", m.key);
    write_linear(o, "transformer.value", m.value);
    write_mlp(o, "transformer.feed_forward", m.feed_forward);
    write_linear(o, "transformer.output", m.output);
    if (m.norm1_gamma) write_vector(o, "transformer.norm1_gamma", *m.norm1_gamma);
    if (m.norm1_beta) write_vector(o, "transformer.norm1_beta", *m.norm1_beta);
    if (m.norm2_gamma) write_vector(o, "transformer.norm2_gamma", *m.norm2_gamma);
    if (m.norm2_beta) write_vector(o, "transformer.norm2_beta", *m.norm2_beta);
    return o.str();
}

void dump_mlp_executor(MlpExecutor& e, const std::string& path, CudaRuntime& rt) {
    MetadataCursor c;
    MlpMetadata m = e.get_meta_data(c);
    Parameters p{e.get_data(rt)};
    RangeValidator r;
    validate_mlp(m, r);
    dump(path, "mlp", mlp_body(m), r.position, p);
}

struct LoadedMlp {
    std::vector<Linear> layers;
    std::optional<std::pair<size_t, size_t>> res;
    Loss loss;
};

LoadedMlp load_mlp_file(const std::string& path, CudaRuntime& rt) {
    Opened o = open_file(path, "mlp");
    MlpMetadata m = read_mlp(need_table(*o.root, "mlp", "checkpoint"), "mlp");
    RangeValidator r;
    validate_mlp(m, r);
    r.finish(o.data_bytes);
    ParameterReader reader(o.data_path, o.data_bytes);
    auto lp = load_mlp_params(m, reader, rt);
    return LoadedMlp{std::move(lp.first), lp.second, m.loss};
}

TransformerMetadata open_transformer(const std::string& path, Opened* out) {
    Opened o = open_file(path, "transformer");
    TransformerMetadata m = read_transformer(need_table(*o.root, "transformer", "checkpoint"),
                                             "transformer");
    RangeValidator r;
    validate_transformer(m, r);
    r.finish(o.data_bytes);
    if (out) *out = std::move(o);
    return m;
}

struct LoadedTransformer {
    Linear q, k, v;
    Matrix position;
    LoadedMlp fcs;
    Linear output;
    NormType norm_type;
    std::optional<Normalization> norm1, norm2;
};

LoadedTransformer load_transformer_file(const std::string& path, CudaRuntime& rt) {
    Opened o;
    TransformerMetadata m = open_transformer(path, &o);
    ParameterReader r(o.data_path, o.data_bytes);
    Linear q = load_linear_params(m.query, r, rt);
    Linear k = load_linear_params(m.key, r, rt);
    Linear v = load_linear_params(m.value, r, rt);
    Matrix pos = rt.matrix_from_host(
        r.read(m.position.byte_start, m.position.byte_end, (uint64_t)m.position.rows * m.position.cols),
        m.position.rows, m.position.cols);
    auto lp = load_mlp_params(m.feed_forward, r, rt);
    Linear out = load_linear_params(m.output, r, rt);
    auto n1 = load_norm(m.normalization, m.norm1_gamma, m.norm1_beta, r, rt);
    auto n2 = load_norm(m.normalization, m.norm2_gamma, m.norm2_beta, r, rt);
    return LoadedTransformer{std::move(q), std::move(k), std::move(v), std::move(pos),
                             LoadedMlp{std::move(lp.first), lp.second, m.feed_forward.loss},
                             std::move(out), m.normalization, std::move(n1), std::move(n2)};
}

void dump_block(InferenceBlock& b, const std::string& path, CudaRuntime& rt) {
    MetadataCursor c;
    TransformerMetadata m = b.get_meta_data(c);
    Parameters p{b.get_data(rt)};
    RangeValidator r;
    validate_transformer(m, r);
    dump(path, "transformer", transformer_body(m), r.position, p);
}

}  // namespace

// ================================================================ public

void dump_linear(Linear& model, const std::string& path, CudaRuntime& rt) {
    MetadataCursor c;
    LinearMetadata m = model.get_meta_data(c);
    Parameters p{model.get_data(rt)};
    RangeValidator r;
    validate_linear(m, r);
    dump(path, "linear", linear_body(m), r.position, p);
}

Linear load_linear(const std::string& path, CudaRuntime& rt) {
    Opened o = open_file(path, "linear");
    LinearMetadata m = read_linear(need_table(*o.root, "linear", "checkpoint"), "linear");
    RangeValidator r;
    validate_linear(m, r);
    r.finish(o.data_bytes);
    ParameterReader reader(o.data_path, o.data_bytes);
    return load_linear_params(m, reader, rt);
}

void dump_mlp(MlpExecutor& model, const std::string& path, CudaRuntime& rt) {
    dump_mlp_executor(model, path, rt);
}
MlpExecutor load_mlp(const std::string& path, CudaRuntime& rt) {
    LoadedMlp l = load_mlp_file(path, rt);
    return MlpExecutor(std::move(l.layers), l.res, l.loss);
}
void dump_inference_mlp(InferenceMLP& model, const std::string& path, CudaRuntime& rt) {
    dump_mlp_executor(model.executor(), path, rt);
}
InferenceMLP load_inference_mlp(const std::string& path, CudaRuntime& rt) {
    LoadedMlp l = load_mlp_file(path, rt);
    return InferenceMLP(std::move(l.layers), l.res, l.loss);
}
void dump_training_mlp(TrainingMlp& model, const std::string& path, CudaRuntime& rt) {
    dump_mlp_executor(model.executor(), path, rt);
}
TrainingMlp load_training_mlp(const std::string& path, CudaRuntime& rt) {
    LoadedMlp l = load_mlp_file(path, rt);
    return TrainingMlp(std::move(l.layers), l.res, l.loss);
}

void dump_transformer(encoder::InferenceTransformer& model, const std::string& path,
                      CudaRuntime& rt) {
    dump_block(model.block(), path, rt);
}

encoder::InferenceTransformer load_transformer(const std::string& path, CudaRuntime& rt) {
    LoadedTransformer t = load_transformer_file(path, rt);
    return encoder::InferenceTransformer(
        std::move(t.q), std::move(t.k), std::move(t.v), std::move(t.position),
        InferenceMLP(std::move(t.fcs.layers), t.fcs.res, t.fcs.loss), std::move(t.output),
        std::nullopt, t.norm_type, std::move(t.norm1), std::move(t.norm2));
}

void dump_training_transformer(encoder::TrainingTransformer& model, const std::string& path,
                               CudaRuntime& rt) {
    MetadataCursor c;
    TransformerMetadata m = model.get_meta_data(c);
    Parameters p{model.get_data(rt)};
    RangeValidator r;
    validate_transformer(m, r);
    dump(path, "transformer", transformer_body(m), r.position, p);
}

encoder::TrainingTransformer load_training_transformer(const std::string& path,
                                                       CudaRuntime& rt) {
    LoadedTransformer t = load_transformer_file(path, rt);
    return encoder::TrainingTransformer(
        std::move(t.q), std::move(t.k), std::move(t.v), std::move(t.position),
        TrainingMlp(std::move(t.fcs.layers), t.fcs.res, t.fcs.loss), std::move(t.output),
        t.norm_type, std::move(t.norm1), std::move(t.norm2));
}

void dump_decoder_transformer(decoder::InferenceTransformer& model, const std::string& path,
                              CudaRuntime& rt) {
    dump_block(model.block(), path, rt);
}

decoder::InferenceTransformer load_decoder_transformer(const std::string& path, CudaRuntime& rt) {
    LoadedTransformer t = load_transformer_file(path, rt);
    decoder::InferenceTransformer model(
        std::move(t.q), std::move(t.k), std::move(t.v), std::move(t.position),
        InferenceMLP(std::move(t.fcs.layers), t.fcs.res, t.fcs.loss), std::move(t.output),
        std::nullopt, t.norm_type);
    if (t.norm1) model.block().attention().normalization() = std::move(*t.norm1);
    if (t.norm2) model.block().norm2() = std::move(*t.norm2);
    return model;
}

std::string inspect(const std::string& path, uint64_t* data_bytes) {
    const std::string meta = metadata_path(path);
    std::unique_ptr<Table> root = Parser(read_text(meta)).parse();
    const std::string type = need_str(*root, "model_type", "checkpoint");
    if (type != "linear" && type != "mlp" && type != "transformer")
        invalid("unknown model type \"" + type + "\"");
    validate_header(*root, type.c_str());
    const uint64_t declared = need_u64(*root, "data_bytes", "checkpoint");
    RangeValidator r;
    if (type == "linear") validate_linear(read_linear(need_table(*root, "linear", "checkpoint"), "linear"), r);
    else if (type == "mlp") validate_mlp(read_mlp(need_table(*root, "mlp", "checkpoint"), "mlp"), r);
    else validate_transformer(read_transformer(need_table(*root, "transformer", "checkpoint"), "transformer"), r);
    r.finish(declared);
    ParameterReader check(resolve_data_path(meta, need_str(*root, "data_file", "checkpoint")),
                          declared);
    if (data_bytes) *data_bytes = declared;
    return type;
}

TransformerMetadata read_transformer_metadata(const std::string& path) {
    return open_transformer(path, nullptr);
}

}  // namespace checkpoint
}  // namespace oxforge
