// cli_json.hpp -- JSON text as nlohmann::json::dump prints it, for the
// command-line drop-ins (their reports are compared byte for byte).
#pragma once

#include <charconv>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <string>

namespace cli_json {

inline std::string quote(const std::string& s)
{
    std::string out = "\"";
    for (const char ch : s) {
        const auto c = static_cast<unsigned char>(ch);
        switch (c) {
        case '"': out += "\\\""; break;
        case '\\': out += "\\\\"; break;
        case '\b': out += "\\b"; break;
        case '\f': out += "\\f"; break;
        case '\n': out += "\\n"; break;
        case '\r': out += "\\r"; break;
        case '\t': out += "\\t"; break;
        default:
            if (c < 0x20) {
                char buf[8];
                std::snprintf(buf, sizeof buf, "\\u%04x", c);
                out += buf;
            } else {
                out += ch;
            }
        }
    }
    return out + "\"";
}

// A finite double as nlohmann::json prints it: the shortest round-trip
// digits d (value = 0.d x 10^n), written in fixed notation when
// -4 < n <= 15 (with ".0" after an integer) and as d.dde+XX otherwise.
inline std::string real(double v)
{
    if (v == 0.0) {
        return std::signbit(v) ? "-0.0" : "0.0";
    }
    char buf[64];
    const auto r = std::to_chars(buf, buf + sizeof buf, v, std::chars_format::scientific);
    const std::string sci(buf, r.ptr);
    std::string sign, digits;
    std::size_t i = 0;
    if (sci[0] == '-') {
        sign = "-";
        i = 1;
    }
    const std::size_t epos = sci.find('e');
    for (std::size_t j = i; j < epos; ++j) {
        if (sci[j] != '.') {
            digits += sci[j];
        }
    }
    const int k = static_cast<int>(digits.size());
    const int n = std::atoi(sci.c_str() + epos + 1) + 1;
    std::string out;
    if (k <= n && n <= 15) {
        out = digits + std::string(static_cast<std::size_t>(n - k), '0') + ".0";
    } else if (0 < n && n <= 15) {
        out = digits.substr(0, static_cast<std::size_t>(n)) + "." +
              digits.substr(static_cast<std::size_t>(n));
    } else if (-4 < n && n <= 0) {
        out = "0." + std::string(static_cast<std::size_t>(-n), '0') + digits;
    } else {
        const int e = n - 1;
        out = digits.substr(0, 1);
        if (k > 1) {
            out += "." + digits.substr(1);
        }
        char eb[8];
        std::snprintf(eb, sizeof eb, "e%c%02d", e < 0 ? '-' : '+', e < 0 ? -e : e);
        out += eb;
    }
    return sign + out;
}

}  // namespace cli_json
