// architecture.json of a Nott checkpoint directory, written and read without
// Boost.
//
// The reference builds the file as a Boost property tree and writes it with
// boost::property_tree::write_json (common/save_load.hpp:3183-3220; the file
// layout in core.hpp:2119-2132: {"name", "modules": [...]}).  A property tree
// node holds a string and an ordered list of (key, child) pairs, and
// write_json prints:
//   * a node without children as its string, quoted (numbers and booleans
//     included: put<int>/put<double>/put<bool> store text);
//   * a node whose children all have empty keys as an array;
//   * any other node as an object;
//   * floating-point values with max_digits10 (17) significant digits,
//     booleans as true/false, and '/' escaped.
// Node below is that tree; descriptor builders restate the per-layer
// serialisers the checkpointed models need (save_load.hpp:2173-2290 layers,
// 2655-2668 residual blocks, 3136-3156 module entries, 601-614 activation
// and initialisation, 2074-2089 local config).  parse() reads any JSON text
// back into the same form (every scalar kept as its text) for Model::load's
// check of the descriptor list (core.hpp:2140-2183).
#pragma once

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <sstream>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace Nott {
namespace HIP {
namespace arch {

struct Node {
    std::string data;
    std::vector<std::pair<std::string, Node>> children;

    Node() = default;
    explicit Node(std::string d) : data(std::move(d)) {}

    // put("a.b", v): the child at the dotted path, created if absent
    // (ptree::put semantics for paths whose components are unique).
    Node& at(const std::string& path) {
        const auto dot = path.find('.');
        const std::string head = path.substr(0, dot);
        Node* child = nullptr;
        for (auto& kv : children)
            if (kv.first == head) child = &kv.second;
        if (!child) {
            children.emplace_back(head, Node{});
            child = &children.back().second;
        }
        return dot == std::string::npos ? *child : child->at(path.substr(dot + 1));
    }
    const Node* find(const std::string& key) const {
        for (auto& kv : children)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
    Node& put(const std::string& path, const std::string& v) { at(path).data = v; return *this; }
    Node& put(const std::string& path, const char* v) { return put(path, std::string(v)); }
    Node& put(const std::string& path, bool v) { return put(path, std::string(v ? "true" : "false")); }
    Node& put(const std::string& path, int64_t v) { return put(path, std::to_string(v)); }
    Node& put(const std::string& path, int v) { return put(path, std::to_string(v)); }
    Node& put(const std::string& path, double v) {
        char buf[40];
        std::snprintf(buf, sizeof buf, "%.17g", v);
        return put(path, std::string(buf));
    }
    Node& add_child(const std::string& path, Node n) { at(path) = std::move(n); return *this; }
    void push_back(Node n) { children.emplace_back(std::string(), std::move(n)); }
    bool is_array() const {
        if (children.empty()) return false;
        for (auto& kv : children)
            if (!kv.first.empty()) return false;
        return true;
    }
};

inline Node int_array(std::initializer_list<int64_t> values) {
    Node a;
    for (int64_t v : values) a.push_back(Node(std::to_string(v)));
    return a;
}

// ------------------------------------------------------------ writer
inline std::string escape(const std::string& s) {
    std::string out;
    for (unsigned char c : s) {
        switch (c) {
            case '"': out += "\\\""; break;
            case '\\': out += "\\\\"; break;
            case '/': out += "\\/"; break;
            case '\b': out += "\\b"; break;
            case '\f': out += "\\f"; break;
            case '\n': out += "\\n"; break;
            case '\r': out += "\\r"; break;
            case '\t': out += "\\t"; break;
            default:
                if (c < 0x20) {
                    char buf[8];
                    std::snprintf(buf, sizeof buf, "\\u%04X", c);
                    out += buf;
                } else {
                    out += static_cast<char>(c);
                }
        }
    }
    return out;
}

inline void write(std::ostream& os, const Node& n, int indent) {
    const std::string pad(4 * indent, ' '), inner(4 * (indent + 1), ' ');
    if (indent > 0 && n.children.empty()) {
        os << '"' << escape(n.data) << '"';
    } else if (indent > 0 && n.is_array()) {
        os << "[\n";
        for (size_t i = 0; i < n.children.size(); ++i) {
            os << inner;
            write(os, n.children[i].second, indent + 1);
            os << (i + 1 < n.children.size() ? ",\n" : "\n");
        }
        os << pad << ']';
    } else {
        os << "{\n";
        for (size_t i = 0; i < n.children.size(); ++i) {
            os << inner << '"' << escape(n.children[i].first) << "\": ";
            write(os, n.children[i].second, indent + 1);
            os << (i + 1 < n.children.size() ? ",\n" : "\n");
        }
        os << pad << '}';
    }
}

inline std::string to_json(const Node& root) {
    std::ostringstream os;
    write(os, root, 0);
    os << '\n';
    return os.str();
}

// ------------------------------------------------------------ reader
class Parser {
public:
    explicit Parser(const std::string& text) : s_(text) {}
    Node parse() {
        Node n = value();
        ws();
        if (i_ != s_.size()) fail("trailing characters");
        return n;
    }

private:
    const std::string& s_;
    size_t i_ = 0;
    [[noreturn]] void fail(const char* what) const {
        throw std::runtime_error(std::string("architecture.json: ") + what + " at offset " + std::to_string(i_));
    }
    void ws() {
        while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\r' || s_[i_] == '\t')) ++i_;
    }
    char peek() { ws(); if (i_ >= s_.size()) fail("unexpected end"); return s_[i_]; }
    void expect(char c) { if (peek() != c) fail("unexpected character"); ++i_; }
    static void utf8(std::string& out, unsigned cp) {
        if (cp < 0x80) { out += static_cast<char>(cp); }
        else if (cp < 0x800) { out += static_cast<char>(0xC0 | (cp >> 6)); out += static_cast<char>(0x80 | (cp & 0x3F)); }
        else {
            out += static_cast<char>(0xE0 | (cp >> 12));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        }
    }
    std::string string() {
        expect('"');
        std::string out;
        while (true) {
            if (i_ >= s_.size()) fail("unterminated string");
            char c = s_[i_++];
            if (c == '"') return out;
            if (c != '\\') { out += c; continue; }
            if (i_ >= s_.size()) fail("unterminated escape");
            char e = s_[i_++];
            switch (e) {
                case '"': case '\\': case '/': out += e; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    if (i_ + 4 > s_.size()) fail("short \\u escape");
                    utf8(out, static_cast<unsigned>(std::strtoul(s_.substr(i_, 4).c_str(), nullptr, 16)));
                    i_ += 4;
                    break;
                }
                default: fail("bad escape");
            }
        }
    }
    Node value() {
        const char c = peek();
        if (c == '{') {
            ++i_;
            Node n;
            if (peek() == '}') { ++i_; return n; }
            while (true) {
                std::string k = string();
                expect(':');
                n.children.emplace_back(std::move(k), value());
                if (peek() == ',') { ++i_; continue; }
                expect('}');
                return n;
            }
        }
        if (c == '[') {
            ++i_;
            Node n;
            if (peek() == ']') { ++i_; return n; }
            while (true) {
                n.push_back(value());
                if (peek() == ',') { ++i_; continue; }
                expect(']');
                return n;
            }
        }
        if (c == '"') return Node(string());
        // a bare number, true, false or null: kept as its text
        const size_t b = i_;
        while (i_ < s_.size() && std::string(",]} \n\r\t").find(s_[i_]) == std::string::npos) ++i_;
        if (b == i_) fail("empty value");
        return Node(s_.substr(b, i_ - b));
    }
};

inline Node parse(const std::string& text) { return Parser(text).parse(); }

inline Node read_file(const std::string& path) {
    std::ifstream f(path);
    if (!f) throw std::runtime_error("Failed to open '" + path + "' for reading.");
    std::stringstream ss;
    ss << f.rdbuf();
    return parse(ss.str());
}

inline void write_file(const std::string& path, const Node& root) {
    std::ofstream f(path);
    if (!f) throw std::runtime_error("Failed to open '" + path + "' for writing.");
    f << to_json(root);
    if (!f) throw std::runtime_error("Failed to write '" + path + "'.");
}

// Leaf equality as the reference's typed reads see it: get<bool> accepts
// true/false and 1/0, get<int64>/get<double> the number's value.
inline bool same_scalar(const std::string& a, const std::string& b) {
    if (a == b) return true;
    auto boolean = [](const std::string& s, int& v) {
        if (s == "true" || s == "1") { v = 1; return true; }
        if (s == "false" || s == "0") { v = 0; return true; }
        return false;
    };
    int ba, bb;
    if (boolean(a, ba) && boolean(b, bb)) return ba == bb;
    char *ea = nullptr, *eb = nullptr;
    const double da = std::strtod(a.c_str(), &ea), db = std::strtod(b.c_str(), &eb);
    return !a.empty() && !b.empty() && *ea == 0 && *eb == 0 && da == db;
}

// True when every field of `want` is present in `got` with the same value
// (arrays element by element, keys looked up by name as the deserialisers
// do; fields `got` holds beyond `want` are ignored, as they are there).
// On a mismatch `where` names the first differing path.
inline bool matches(const Node& want, const Node& got, std::string& where, const std::string& path = "") {
    if (want.children.empty()) {
        if (!got.children.empty() || !same_scalar(want.data, got.data)) { where = path; return false; }
        return true;
    }
    if (want.is_array()) {
        if (got.children.size() != want.children.size()) { where = path; return false; }
        for (size_t i = 0; i < want.children.size(); ++i)
            if (!matches(want.children[i].second, got.children[i].second, where, path + "[" + std::to_string(i) + "]"))
                return false;
        return true;
    }
    for (auto& kv : want.children) {
        const Node* g = got.find(kv.first);
        const std::string p = path.empty() ? kv.first : path + "." + kv.first;
        if (!g) { where = p; return false; }
        if (!matches(kv.second, *g, where, p)) return false;
    }
    return true;
}

// ------------------------------------------------------------ descriptors
// Layer descriptors with the fields the reference's serialiser writes for
// them (save_load.hpp:2173-2290), default values from the descriptor
// structs (conv.hpp:39-49, fc.hpp:19-28, batchnorm.hpp:22-33,
// pooling.hpp:41-63, flatten.hpp:14-17, activation.hpp:23-25,
// initialization.hpp:17-19).
inline Node typed(const char* type) { Node n; n.put("type", type); return n; }
inline Node local_config() { Node n; n.add_child("regularization", Node{}); return n; }

inline Node conv2d(int64_t cin, int64_t cout, int64_t k, int64_t stride, int64_t pad, bool bias,
                   const char* activation, const char* init) {
    Node d = typed("conv2d");
    d.put("options.in_channels", cin);
    d.put("options.out_channels", cout);
    d.add_child("options.kernel_size", int_array({k, k}));
    d.add_child("options.stride", int_array({stride, stride}));
    d.add_child("options.padding", int_array({pad, pad}));
    d.add_child("options.dilation", int_array({1, 1}));
    d.put("options.groups", int64_t{1});
    d.put("options.bias", bias);
    d.put("options.padding_mode", "zeros");
    d.add_child("activation", typed(activation));
    d.add_child("initialization", typed(init));
    d.add_child("local", local_config());
    return d;
}

inline Node fc(int64_t in, int64_t out, bool bias, const char* activation, const char* init) {
    Node d = typed("fc");
    d.put("options.in_features", in);
    d.put("options.out_features", out);
    d.put("options.bias", bias);
    d.add_child("activation", typed(activation));
    d.add_child("initialization", typed(init));
    d.add_child("local", local_config());
    return d;
}

inline Node batch_norm2d(int64_t features, const char* activation) {
    Node d = typed("batch_norm2d");
    d.put("options.num_features", features);
    d.put("options.eps", 1e-5);
    d.put("options.momentum", 0.1);
    d.put("options.affine", true);
    d.put("options.track_running_stats", true);
    d.add_child("activation", typed(activation));
    d.add_child("initialization", typed("default"));
    d.add_child("local", local_config());
    return d;
}

inline Node max_pool2d(int64_t k, int64_t stride, int64_t pad) {
    Node d = typed("pooling");
    d.put("options.variant", "max2d");
    d.add_child("options.kernel_size", int_array({k, k}));
    d.add_child("options.stride", int_array({stride, stride}));
    d.add_child("options.padding", int_array({pad, pad}));
    d.add_child("options.dilation", int_array({1, 1}));
    d.put("options.ceil_mode", false);
    d.add_child("activation", typed("identity"));
    d.add_child("local", local_config());
    return d;
}

inline Node adaptive_avg_pool2d(int64_t h, int64_t w) {
    Node d = typed("pooling");
    d.put("options.variant", "adaptive_avg2d");
    d.add_child("options.output_size", int_array({h, w}));
    d.add_child("activation", typed("identity"));
    d.add_child("local", local_config());
    return d;
}

inline Node flatten(int64_t start_dim = 1, int64_t end_dim = -1) {
    Node d = typed("flatten");
    d.put("options.start_dim", start_dim);
    d.put("options.end_dim", end_dim);
    d.add_child("activation", typed("identity"));
    d.add_child("local", local_config());
    return d;
}

// Residual block descriptor (save_load.hpp:2655-2668).
inline Node residual(std::vector<Node> layers, const Node* projection, const char* final_activation,
                     int64_t repeats = 1, double dropout = 0.0) {
    Node d = typed("residual");
    Node ls;
    for (auto& l : layers) ls.push_back(std::move(l));
    d.add_child("layers", std::move(ls));
    d.put("repeats", repeats);
    if (projection) d.add_child("skip.projection", *projection);
    d.add_child("output.final_activation", typed(final_activation));
    d.put("output.dropout", dropout);
    d.add_child("local", local_config());
    return d;
}

// A "modules" entry (save_load.hpp:3136-3156): kind layer/block, the
// descriptor, and the module's name when it has one.
inline Node module(const char* kind, Node descriptor, const std::string& name = {}) {
    Node m;
    m.put("kind", kind);
    m.add_child("descriptor", std::move(descriptor));
    if (!name.empty()) m.put("name", name);
    return m;
}

// The whole file (core.hpp:2122-2123).
inline Node architecture(const std::string& name, std::vector<Node> modules) {
    Node root;
    root.put("name", name);
    Node list;
    for (auto& m : modules) list.push_back(std::move(m));
    root.add_child("modules", std::move(list));
    return root;
}

}  // namespace arch
}  // namespace HIP
}  // namespace Nott
