// Minimal JSON reader for index.json and load options: objects, arrays, strings (with escapes),
// numbers, booleans and null. Throws qne::Error(QNE_EFORMAT) on malformed input.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "error.hpp"

namespace qne {

struct Json {
    enum Type { Null, Bool, Number, String, Array, Object } type = Null;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Json> arr;
    std::map<std::string, Json> obj;

    bool has(const std::string& k) const { return type == Object && obj.count(k) != 0; }
    const Json& at(const std::string& k) const {
        if (type != Object) throw Error(QNE_EFORMAT, "expected a JSON object looking up '" + k + "'");
        auto it = obj.find(k);
        if (it == obj.end()) throw Error(QNE_EFORMAT, "missing key '" + k + "'");
        return it->second;
    }
    double number() const {
        if (type != Number) throw Error(QNE_EFORMAT, "expected a number");
        return num;
    }
    // Non-negative integer that fits in 64 bits, exactly represented.
    uint64_t u64(const std::string& what) const {
        if (type != Number || num < 0 || num != (double)(uint64_t)num || num > 9.007199254740992e15)
            throw Error(QNE_EFORMAT, "expected a non-negative integer for " + what);
        return (uint64_t)num;
    }
    const std::string& string() const {
        if (type != String) throw Error(QNE_EFORMAT, "expected a string");
        return str;
    }

    static Json parse(const char* s, size_t n) {
        Parser p{s, s + n};
        p.ws();
        Json v = p.value(0);
        p.ws();
        if (p.p != p.e) throw Error(QNE_EFORMAT, "trailing characters after JSON value");
        return v;
    }

  private:
    struct Parser {
        const char* p;
        const char* e;
        void ws() {
            while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) p++;
        }
        [[noreturn]] void fail(const char* what) { throw Error(QNE_EFORMAT, std::string("index.json: ") + what); }
        bool lit(const char* t) {
            size_t n = 0;
            while (t[n]) n++;
            if ((size_t)(e - p) < n) return false;
            for (size_t i = 0; i < n; i++)
                if (p[i] != t[i]) return false;
            p += n;
            return true;
        }
        static void utf8(std::string& out, uint32_t cp) {
            if (cp < 0x80) out += (char)cp;
            else if (cp < 0x800) { out += (char)(0xC0 | (cp >> 6)); out += (char)(0x80 | (cp & 63)); }
            else if (cp < 0x10000) { out += (char)(0xE0 | (cp >> 12)); out += (char)(0x80 | ((cp >> 6) & 63)); out += (char)(0x80 | (cp & 63)); }
            else { out += (char)(0xF0 | (cp >> 18)); out += (char)(0x80 | ((cp >> 12) & 63)); out += (char)(0x80 | ((cp >> 6) & 63)); out += (char)(0x80 | (cp & 63)); }
        }
        uint32_t hex4() {
            if (e - p < 4) fail("short \\u escape");
            uint32_t v = 0;
            for (int i = 0; i < 4; i++) {
                char c = *p++;
                v <<= 4;
                if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
                else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
                else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
                else fail("bad \\u escape");
            }
            return v;
        }
        std::string strv() {
            std::string out;
            p++;  // opening quote
            while (true) {
                if (p >= e) fail("unterminated string");
                char c = *p++;
                if (c == '"') break;
                if ((unsigned char)c < 0x20) fail("control character in string");
                if (c != '\\') { out += c; continue; }
                if (p >= e) fail("unterminated escape");
                char x = *p++;
                switch (x) {
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
                        if (cp >= 0xD800 && cp < 0xDC00 && e - p >= 6 && p[0] == '\\' && p[1] == 'u') {
                            p += 2;
                            uint32_t lo = hex4();
                            if (lo < 0xDC00 || lo >= 0xE000) fail("bad surrogate pair");
                            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                        }
                        utf8(out, cp);
                        break;
                    }
                    default: fail("bad escape");
                }
            }
            return out;
        }
        Json value(int depth) {
            if (depth > 64) fail("nesting too deep");
            if (p >= e) fail("unexpected end");
            Json v;
            char c = *p;
            if (c == '{') {
                v.type = Object;
                p++;
                ws();
                if (p < e && *p == '}') { p++; return v; }
                while (true) {
                    ws();
                    if (p >= e || *p != '"') fail("expected a key");
                    std::string k = strv();
                    ws();
                    if (p >= e || *p != ':') fail("expected ':'");
                    p++;
                    ws();
                    v.obj[k] = value(depth + 1);
                    ws();
                    if (p < e && *p == ',') { p++; continue; }
                    if (p < e && *p == '}') { p++; break; }
                    fail("expected ',' or '}'");
                }
            } else if (c == '[') {
                v.type = Array;
                p++;
                ws();
                if (p < e && *p == ']') { p++; return v; }
                while (true) {
                    ws();
                    v.arr.push_back(value(depth + 1));
                    ws();
                    if (p < e && *p == ',') { p++; continue; }
                    if (p < e && *p == ']') { p++; break; }
                    fail("expected ',' or ']'");
                }
            } else if (c == '"') {
                v.type = String;
                v.str = strv();
            } else if (lit("true")) { v.type = Bool; v.b = true; }
            else if (lit("false")) { v.type = Bool; v.b = false; }
            else if (lit("null")) { v.type = Null; }
            else {
                const char* start = p;
                if (p < e && (*p == '-' || *p == '+')) p++;
                while (p < e && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '-' || *p == '+')) p++;
                if (p == start) fail("unexpected character");
                std::string t(start, p);
                char* end = nullptr;
                v.num = std::strtod(t.c_str(), &end);
                if (!end || *end) fail("bad number");
                v.type = Number;
            }
            return v;
        }
    };
};

}  // namespace qne
