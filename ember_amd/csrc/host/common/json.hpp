// A JSON document model for the three files the backend reads: config.json,
// generation_config.json and a safetensors header. The public declarations are
// the reference's (src/common/json.hpp:15-92), so ModelConfig::from_json and
// its callers keep their signatures; the representation below and every
// definition (json.cpp) are this build's.
//
// An object keeps its members in document order and finds a key by a linear
// scan: these documents hold at most a few thousand members.
#pragma once

#include <cstdint>
#include <string>
#include <string_view>
#include <utility>
#include <vector>

namespace ember::json {

class Value;
using Array = std::vector<Value>;
using Object = std::vector<std::pair<std::string, Value>>;

class Value {
public:
    enum class Type { null, boolean, number, string, array, object };

    Value() = default;
    Value(std::nullptr_t) {}
    Value(bool b) : kind_(Type::boolean), truth_(b) {}
    Value(double d) : kind_(Type::number), real_(d) {}
    Value(int i) : Value(static_cast<int64_t>(i)) {}
    Value(int64_t i) : kind_(Type::number), exact_(true), real_(static_cast<double>(i)), whole_(i) {}
    Value(uint64_t i);  // exact when it fits int64_t, else held as a double
    Value(const char *s) : kind_(Type::string), text_(s) {}
    Value(std::string s) : kind_(Type::string), text_(std::move(s)) {}
    Value(std::string_view s) : kind_(Type::string), text_(s) {}
    Value(Array a) : kind_(Type::array), items_(std::move(a)) {}
    Value(Object o) : kind_(Type::object), members_(std::move(o)) {}

    // Throws ember::Error naming the line and column of the first problem.
    static Value parse(std::string_view text);

    Type type() const { return kind_; }
    bool is_null() const { return type() == Type::null; }
    bool is_bool() const { return type() == Type::boolean; }
    bool is_number() const { return type() == Type::number; }
    bool is_string() const { return type() == Type::string; }
    bool is_array() const { return type() == Type::array; }
    bool is_object() const { return type() == Type::object; }

    // Typed access; each throws ember::Error on a type mismatch.
    bool as_bool() const;
    double as_number() const;
    int64_t as_int() const;  // also throws for a number with a fraction
    const std::string &as_string() const;
    const Array &as_array() const;
    const Object &as_object() const;
    Array &as_array();
    Object &as_object();

    // Object members.
    const Value *find(std::string_view key) const;        // nullptr when absent or not an object
    const Value &operator[](std::string_view key) const;  // throws when absent
    bool contains(std::string_view key) const { return find(key) != nullptr; }
    Value &set(std::string_view key, Value value);        // a null value becomes an object

    // Optional members with defaults.
    double get_number(std::string_view key, double def) const;
    int64_t get_int(std::string_view key, int64_t def) const;
    bool get_bool(std::string_view key, bool def) const;
    std::string get_string(std::string_view key, std::string_view def) const;

    // Array elements.
    size_t size() const;
    const Value &operator[](size_t i) const;
    void push(Value value);  // a null value becomes an array

    std::string dump() const;
    void dump_to(std::string &out) const;

private:
    // Throws unless this value is of kind `want`; `what` names the access.
    void require(Type want, const char *what) const;

    // One flat record: `kind_` says which of the fields after it holds the value.
    Type kind_ = Type::null;
    bool truth_ = false;   // boolean
    bool exact_ = false;   // number: the text was an integer that fits int64_t, kept in whole_
    double real_ = 0.0;    // number, as a double (always set)
    int64_t whole_ = 0;    // number, exactly, when exact_
    std::string text_;     // string
    Array items_;          // array
    Object members_;       // object members, in document order
};

// Appends s as a JSON string literal.
void write_string(std::string &out, std::string_view s);

}  // namespace ember::json
