// JSON for the declarations in json.hpp: a recursive-descent parser over the
// text (RFC 8259: objects, arrays, strings with escapes and surrogate pairs,
// numbers, literals), the typed accessors over Value's flat record, and a
// compact writer.
#include "common/json.hpp"

#include <algorithm>
#include <charconv>
#include <cmath>
#include <cstdio>
#include <cstdlib>

#include "common/error.hpp"

namespace ember::json {

namespace {

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

// How messages name each kind, indexed by Value::Type.
constexpr const char *kKindNames[] = {"null", "a boolean", "a number", "a string", "an array", "an object"};

const char *kind_name(Value::Type t) { return kKindNames[static_cast<size_t>(t)]; }

// An optional member: absent or null gives the fallback; otherwise `read` converts it (and checks its kind).
template <class T, class Read>
T member_or(const Value &object, std::string_view key, T fallback, Read read) {
    const Value *member = object.find(key);
    return member == nullptr || member->is_null() ? fallback : read(*member);
}

// Integers print exactly; other numbers with 17 significant digits, which round-trip a double. JSON has no
// infinities or NaNs, so those print as null.
void append_number(std::string &out, bool exact, int64_t whole, double real) {
    char buf[32];
    if (exact) {
        const auto res = std::to_chars(buf, buf + sizeof buf, whole);
        out.append(buf, res.ptr);
    } else if (std::isfinite(real)) {
        out.append(buf, static_cast<size_t>(std::snprintf(buf, sizeof buf, "%.17g", real)));
    } else {
        out += "null";
    }
}

}  // namespace

Value Value::parse(std::string_view text) { return Parser(text).document(); }

Value::Value(uint64_t i) : kind_(Type::number), real_(static_cast<double>(i)) {
    if (i <= static_cast<uint64_t>(INT64_MAX)) {
        exact_ = true;
        whole_ = static_cast<int64_t>(i);
    }
}

void Value::require(Type want, const char *what) const {
    if (kind_ != want) fail("JSON: {} needs {}, but the value is {}", what, kind_name(want), kind_name(kind_));
}

bool Value::as_bool() const {
    require(Type::boolean, "as_bool");
    return truth_;
}

double Value::as_number() const {
    require(Type::number, "as_number");
    return real_;
}

int64_t Value::as_int() const {
    require(Type::number, "as_int");
    if (exact_) return whole_;
    // Written with a fraction or an exponent ("2.0", "1e3"): still an integer if the value is whole and in range.
    constexpr double kTwo63 = 9223372036854775808.0;
    if (std::nearbyint(real_) == real_ && real_ >= -kTwo63 && real_ < kTwo63) return static_cast<int64_t>(real_);
    fail("JSON: as_int needs a whole number, but the value is {}", real_);
}

const std::string &Value::as_string() const {
    require(Type::string, "as_string");
    return text_;
}

const Array &Value::as_array() const {
    require(Type::array, "as_array");
    return items_;
}

const Object &Value::as_object() const {
    require(Type::object, "as_object");
    return members_;
}

Array &Value::as_array() {
    require(Type::array, "as_array");
    return items_;
}

Object &Value::as_object() {
    require(Type::object, "as_object");
    return members_;
}

const Value *Value::find(std::string_view key) const {
    if (kind_ != Type::object) return nullptr;
    const auto hit = std::find_if(members_.begin(), members_.end(), [key](const auto &m) { return m.first == key; });
    return hit == members_.end() ? nullptr : &hit->second;
}

const Value &Value::operator[](std::string_view key) const {
    if (const Value *member = find(key)) return *member;
    fail("JSON: no member named \"{}\"", key);
}

Value &Value::set(std::string_view key, Value value) {
    if (kind_ == Type::null) kind_ = Type::object;
    require(Type::object, "set");
    auto slot = std::find_if(members_.begin(), members_.end(), [key](const auto &m) { return m.first == key; });
    if (slot == members_.end()) slot = members_.insert(members_.end(), {std::string(key), Value()});
    slot->second = std::move(value);
    return slot->second;
}

double Value::get_number(std::string_view key, double def) const {
    return member_or(*this, key, def, [](const Value &v) { return v.as_number(); });
}

int64_t Value::get_int(std::string_view key, int64_t def) const {
    return member_or(*this, key, def, [](const Value &v) { return v.as_int(); });
}

bool Value::get_bool(std::string_view key, bool def) const {
    return member_or(*this, key, def, [](const Value &v) { return v.as_bool(); });
}

std::string Value::get_string(std::string_view key, std::string_view def) const {
    return member_or(*this, key, std::string(def), [](const Value &v) { return v.as_string(); });
}

size_t Value::size() const {
    if (kind_ == Type::array) return items_.size();
    if (kind_ == Type::object) return members_.size();
    fail("JSON: size needs an array or an object, but the value is {}", kind_name(kind_));
}

const Value &Value::operator[](size_t i) const {
    require(Type::array, "operator[](index)");
    if (i < items_.size()) return items_[i];
    fail("JSON: index {} is past the end of an array of {} elements", i, items_.size());
}

void Value::push(Value value) {
    if (kind_ == Type::null) kind_ = Type::array;
    require(Type::array, "push");
    items_.push_back(std::move(value));
}

void write_string(std::string &out, std::string_view s) {
    // Short escapes of the control characters 0x08..0x0D (0x0B has none).
    constexpr char kShort[] = {'b', 't', 'n', 0, 'f', 'r'};
    out.push_back('"');
    for (const char ch : s) {
        const auto c = static_cast<unsigned char>(ch);
        if (c == '"' || c == '\\') {
            out.push_back('\\');
            out.push_back(ch);
        } else if (c >= 0x20) {
            out.push_back(ch);
        } else if (c >= 0x08 && c <= 0x0D && kShort[c - 0x08] != 0) {
            out.push_back('\\');
            out.push_back(kShort[c - 0x08]);
        } else {
            char buf[8];
            out.append(buf, static_cast<size_t>(std::snprintf(buf, sizeof buf, "\\u%04x", static_cast<unsigned>(c))));
        }
    }
    out.push_back('"');
}

void Value::dump_to(std::string &out) const {
    switch (kind_) {
        case Type::null:
            out += "null";
            return;
        case Type::boolean:
            out += truth_ ? "true" : "false";
            return;
        case Type::number:
            append_number(out, exact_, whole_, real_);
            return;
        case Type::string:
            write_string(out, text_);
            return;
        case Type::array:
            out.push_back('[');
            for (size_t i = 0; i < items_.size(); ++i) {
                if (i > 0) out.push_back(',');
                items_[i].dump_to(out);
            }
            out.push_back(']');
            return;
        case Type::object:
            out.push_back('{');
            for (size_t i = 0; i < members_.size(); ++i) {
                if (i > 0) out.push_back(',');
                write_string(out, members_[i].first);
                out.push_back(':');
                members_[i].second.dump_to(out);
            }
            out.push_back('}');
            return;
    }
}

std::string Value::dump() const {
    std::string out;
    dump_to(out);
    return out;
}

}  // namespace ember::json
