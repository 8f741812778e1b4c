// Errors of the host side. Same contract as the reference's
// src/common/error.hpp:1-25 (ember::Error, fail(), EMBER_CHECK), without
// <format>, which this toolchain's standard libraries do not ship: messages use
// "{}" placeholders filled left to right through an ostream.
#pragma once

#include <sstream>
#include <stdexcept>
#include <string>

namespace ember {

class Error : public std::runtime_error {
public:
    explicit Error(const std::string &msg) : std::runtime_error(msg) {}
};

namespace detail {

inline void format_into(std::ostringstream &os, const char *fmt) { os << fmt; }

template <class A, class... Rest>
void format_into(std::ostringstream &os, const char *fmt, const A &a, const Rest &...rest) {
    for (const char *p = fmt; *p; p++) {
        if (p[0] == '{' && p[1] == '}') {
            os << a;
            format_into(os, p + 2, rest...);
            return;
        }
        os << *p;
    }
}

}  // namespace detail

template <class... Args>
std::string format(const char *fmt, const Args &...args) {
    std::ostringstream os;
    detail::format_into(os, fmt, args...);
    return os.str();
}

template <class... Args>
[[noreturn]] void fail(const char *fmt, const Args &...args) {
    throw Error(format(fmt, args...));
}

#define EMBER_CHECK(cond, ...)                   \
    do {                                         \
        if (!(cond)) ::ember::fail(__VA_ARGS__); \
    } while (0)

}  // namespace ember
