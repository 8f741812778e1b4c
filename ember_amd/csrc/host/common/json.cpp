// JSON parsing and serialization for the declarations in json.hpp: a
// recursive-descent parser over the text (RFC 8259: objects, arrays, strings
// with escapes and surrogate pairs, numbers, literals), and a writer.
#include "common/json.hpp"

#include <charconv>
#include <cmath>
#include <cstdio>
#include <cstdlib>

#include "common/error.hpp"

namespace ember::json {

namespace {

const char *type_name(Value::Type t) {
    switch (t) {
        case Value::Type::null: return "null";
        case Value::Type::boolean: return "a boolean";
        case Value::Type::number: return "a number";
        case Value::Type::string: return "a string";
        case Value::Type::array: return "an array";
        case Value::Type::object: return "an object";
    }
    return "?";
}

class Parser {
public:
    explicit Parser(std::string_view text) : s_(text) {}

    Value document() {
        Value v = value(0);
        skip_space();
        if (at_ < s_.size()) error("unexpected text after the value");
        return v;
    }

private:
    static constexpr int kMaxDepth = 512;

    [[noreturn]] void error(const char *what) const {
        int line = 1, col = 1;
        for (size_t i = 0; i < at_ && i < s_.size(); i++) {
            if (s_[i] == '\n') {
                line++;
                col = 1;
            } else {
                col++;
            }
        }
        fail("JSON: {} at line {}, column {}", what, line, col);
    }

    void skip_space() {
        while (at_ < s_.size() && (s_[at_] == ' ' || s_[at_] == '\t' || s_[at_] == '\n' || s_[at_] == '\r')) at_++;
    }

    bool take(char c) {
        skip_space();
        if (at_ < s_.size() && s_[at_] == c) {
            at_++;
            return true;
        }
        return false;
    }

    void expect(char c, const char *what) {
        if (!take(c)) error(what);
    }

    bool literal(std::string_view word) {
        if (s_.substr(at_, word.size()) == word) {
            at_ += word.size();
            return true;
        }
        return false;
    }

    Value value(int depth) {
        if (depth > kMaxDepth) error("nesting too deep");
        skip_space();
        if (at_ >= s_.size()) error("unexpected end of text");
        const char c = s_[at_];
        if (c == '{') return object(depth);
        if (c == '[') return array(depth);
        if (c == '"') return Value(string());
        if (c == '-' || (c >= '0' && c <= '9')) return number();
        if (literal("true")) return Value(true);
        if (literal("false")) return Value(false);
        if (literal("null")) return Value();
        error("expected a value");
    }

    Value object(int depth) {
        at_++;  // '{'
        Object members;
        if (take('}')) return Value(std::move(members));
        do {
            skip_space();
            if (at_ >= s_.size() || s_[at_] != '"') error("expected a member name");
            std::string key = string();
            expect(':', "expected ':' after a member name");
            members.emplace_back(std::move(key), value(depth + 1));
        } while (take(','));
        expect('}', "expected ',' or '}' in an object");
        return Value(std::move(members));
    }

    Value array(int depth) {
        at_++;  // '['
        Array items;
        if (take(']')) return Value(std::move(items));
        do {
            items.push_back(value(depth + 1));
        } while (take(','));
        expect(']', "expected ',' or ']' in an array");
        return Value(std::move(items));
    }

    unsigned hex4() {
        if (at_ + 4 > s_.size()) error("truncated \\u escape");
        unsigned v = 0;
        for (int i = 0; i < 4; i++) {
            const char c = s_[at_++];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= static_cast<unsigned>(c - '0');
            else if (c >= 'a' && c <= 'f') v |= static_cast<unsigned>(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= static_cast<unsigned>(c - 'A' + 10);
            else error("bad hex digit in a \\u escape");
        }
        return v;
    }

    static void put_utf8(std::string &out, unsigned cp) {
        if (cp < 0x80) {
            out += static_cast<char>(cp);
        } else if (cp < 0x800) {
            out += static_cast<char>(0xC0 | (cp >> 6));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += static_cast<char>(0xE0 | (cp >> 12));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        } else {
            out += static_cast<char>(0xF0 | (cp >> 18));
            out += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        }
    }

    std::string string() {
        at_++;  // '"'
        std::string out;
        for (;;) {
            if (at_ >= s_.size()) error("unterminated string");
            const char c = s_[at_++];
            if (c == '"') return out;
            if (static_cast<unsigned char>(c) < 0x20) error("control character in a string");
            if (c != '\\') {
                out += c;
                continue;
            }
            if (at_ >= s_.size()) error("unterminated escape");
            const char e = s_[at_++];
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
                    unsigned cp = hex4();
                    if (cp >= 0xD800 && cp < 0xDC00) {  // a high surrogate needs its low half
                        if (at_ + 2 > s_.size() || s_[at_] != '\\' || s_[at_ + 1] != 'u') error("unpaired surrogate");
                        at_ += 2;
                        const unsigned lo = hex4();
                        if (lo < 0xDC00 || lo >= 0xE000) error("unpaired surrogate");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp < 0xE000) {
                        error("unpaired surrogate");
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: error("unknown escape");
            }
        }
    }

    Value number() {
        const size_t start = at_;
        bool integral = true;
        if (s_[at_] == '-') at_++;
        auto digits = [&] {
            const size_t d0 = at_;
            while (at_ < s_.size() && s_[at_] >= '0' && s_[at_] <= '9') at_++;
            if (at_ == d0) error("expected digits");
        };
        digits();
        if (at_ < s_.size() && s_[at_] == '.') {
            integral = false;
            at_++;
            digits();
        }
        if (at_ < s_.size() && (s_[at_] == 'e' || s_[at_] == 'E')) {
            integral = false;
            at_++;
            if (at_ < s_.size() && (s_[at_] == '+' || s_[at_] == '-')) at_++;
            digits();
        }
        const std::string_view text = s_.substr(start, at_ - start);
        if (integral) {
            int64_t i = 0;
            auto [end, ec] = std::from_chars(text.data(), text.data() + text.size(), i);
            if (ec == std::errc() && end == text.data() + text.size()) return Value(i);
        }
        const std::string copy(text);  // strtod needs a terminated string
        return Value(std::strtod(copy.c_str(), nullptr));
    }

    std::string_view s_;
    size_t at_ = 0;
};

}  // namespace

Value Value::parse(std::string_view text) { return Parser(text).document(); }

bool Value::as_bool() const {
    if (!is_bool()) fail("JSON: expected a boolean, found {}", type_name(type()));
    return std::get<bool>(v_);
}

double Value::as_number() const {
    if (!is_number()) fail("JSON: expected a number, found {}", type_name(type()));
    return std::get<Number>(v_).d;
}

int64_t Value::as_int() const {
    if (!is_number()) fail("JSON: expected an integer, found {}", type_name(type()));
    const Number &n = std::get<Number>(v_);
    if (n.is_int) return n.i;
    if (std::trunc(n.d) != n.d || std::fabs(n.d) > 9.2e18) fail("JSON: expected an integer, found {}", n.d);
    return static_cast<int64_t>(n.d);
}

const std::string &Value::as_string() const {
    if (!is_string()) fail("JSON: expected a string, found {}", type_name(type()));
    return std::get<std::string>(v_);
}

const Array &Value::as_array() const {
    if (!is_array()) fail("JSON: expected an array, found {}", type_name(type()));
    return std::get<Array>(v_);
}

const Object &Value::as_object() const {
    if (!is_object()) fail("JSON: expected an object, found {}", type_name(type()));
    return std::get<Object>(v_);
}

Array &Value::as_array() {
    if (!is_array()) fail("JSON: expected an array, found {}", type_name(type()));
    return std::get<Array>(v_);
}

Object &Value::as_object() {
    if (!is_object()) fail("JSON: expected an object, found {}", type_name(type()));
    return std::get<Object>(v_);
}

const Value *Value::find(std::string_view key) const {
    if (!is_object()) return nullptr;
    for (const auto &[k, v] : std::get<Object>(v_))
        if (k == key) return &v;
    return nullptr;
}

const Value &Value::operator[](std::string_view key) const {
    const Value *v = find(key);
    if (!v) fail("JSON: missing member \"{}\"", std::string(key));
    return *v;
}

Value &Value::set(std::string_view key, Value value) {
    if (is_null()) v_ = Object{};
    Object &o = as_object();
    for (auto &[k, v] : o)
        if (k == key) return v = std::move(value);
    o.emplace_back(std::string(key), std::move(value));
    return o.back().second;
}

double Value::get_number(std::string_view key, double def) const {
    const Value *v = find(key);
    return v && !v->is_null() ? v->as_number() : def;
}

int64_t Value::get_int(std::string_view key, int64_t def) const {
    const Value *v = find(key);
    return v && !v->is_null() ? v->as_int() : def;
}

bool Value::get_bool(std::string_view key, bool def) const {
    const Value *v = find(key);
    return v && !v->is_null() ? v->as_bool() : def;
}

std::string Value::get_string(std::string_view key, std::string_view def) const {
    const Value *v = find(key);
    return v && !v->is_null() ? v->as_string() : std::string(def);
}

size_t Value::size() const {
    if (is_array()) return std::get<Array>(v_).size();
    if (is_object()) return std::get<Object>(v_).size();
    fail("JSON: size() of {}", type_name(type()));
}

const Value &Value::operator[](size_t i) const {
    const Array &a = as_array();
    if (i >= a.size()) fail("JSON: index {} past an array of {}", i, a.size());
    return a[i];
}

void Value::push(Value value) {
    if (is_null()) v_ = Array{};
    as_array().push_back(std::move(value));
}

void write_string(std::string &out, std::string_view s) {
    out += '"';
    for (const char c : s) {
        switch (c) {
            case '"': out += "\\\""; break;
            case '\\': out += "\\\\"; break;
            case '\n': out += "\\n"; break;
            case '\r': out += "\\r"; break;
            case '\t': out += "\\t"; break;
            case '\b': out += "\\b"; break;
            case '\f': out += "\\f"; break;
            default:
                if (static_cast<unsigned char>(c) < 0x20) {
                    char buf[8];
                    std::snprintf(buf, sizeof buf, "\\u%04x", static_cast<unsigned>(static_cast<unsigned char>(c)));
                    out += buf;
                } else {
                    out += c;
                }
        }
    }
    out += '"';
}

void Value::dump_to(std::string &out) const {
    switch (type()) {
        case Type::null: out += "null"; break;
        case Type::boolean: out += std::get<bool>(v_) ? "true" : "false"; break;
        case Type::number: {
            const Number &n = std::get<Number>(v_);
            char buf[32];
            if (n.is_int) {
                std::snprintf(buf, sizeof buf, "%lld", static_cast<long long>(n.i));
            } else if (!std::isfinite(n.d)) {
                std::snprintf(buf, sizeof buf, "null");  // JSON has no inf / nan
            } else {
                std::snprintf(buf, sizeof buf, "%.17g", n.d);
            }
            out += buf;
            break;
        }
        case Type::string: write_string(out, std::get<std::string>(v_)); break;
        case Type::array: {
            out += '[';
            bool first = true;
            for (const Value &v : std::get<Array>(v_)) {
                if (!first) out += ',';
                first = false;
                v.dump_to(out);
            }
            out += ']';
            break;
        }
        case Type::object: {
            out += '{';
            bool first = true;
            for (const auto &[k, v] : std::get<Object>(v_)) {
                if (!first) out += ',';
                first = false;
                write_string(out, k);
                out += ':';
                v.dump_to(out);
            }
            out += '}';
            break;
        }
    }
}

std::string Value::dump() const {
    std::string out;
    dump_to(out);
    return out;
}

}  // namespace ember::json
