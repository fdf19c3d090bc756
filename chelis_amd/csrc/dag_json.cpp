// JSON values for the DAG front end: a recursive-descent reader (RFC 8259
// grammar, nesting limited to 256) and a compact writer. Numbers keep their
// spelling so 64-bit integers pass through exactly.
#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "dag.h"

namespace chelis {
namespace dag {

const Json *Json::get(const char *key) const {
    if (kind != Object) return nullptr;
    for (const auto &f : fields)
        if (f.first == key) return &f.second;
    return nullptr;
}

bool Json::is_int() const {
    if (kind != Number || text.empty()) return false;
    size_t i = text[0] == '-' ? 1 : 0;
    if (i >= text.size()) return false;
    for (; i < text.size(); ++i)
        if (text[i] < '0' || text[i] > '9') return false;
    errno = 0;
    (void)std::strtoll(text.c_str(), nullptr, 10);
    return errno == 0;
}

int64_t Json::as_int() const { return std::strtoll(text.c_str(), nullptr, 10); }

double Json::as_double() const { return std::strtod(text.c_str(), nullptr); }

namespace {

struct Reader {
    const char *s;
    size_t n, i = 0;
    std::string error;

    bool fail(const char *what) {
        if (error.empty()) error = std::string(what) + " at byte " + std::to_string(i);
        return false;
    }
    void space() {
        while (i < n && (s[i] == ' ' || s[i] == '\t' || s[i] == '\n' || s[i] == '\r')) ++i;
    }
    bool literal(const char *word) {
        const size_t len = std::strlen(word);
        if (n - i < len || std::memcmp(s + i, word, len) != 0) return fail("invalid literal");
        i += len;
        return true;
    }
    static void put_utf8(std::string *out, uint32_t cp) {
        if (cp < 0x80) {
            out->push_back((char)cp);
        } else if (cp < 0x800) {
            out->push_back((char)(0xC0 | (cp >> 6)));
            out->push_back((char)(0x80 | (cp & 0x3F)));
        } else if (cp < 0x10000) {
            out->push_back((char)(0xE0 | (cp >> 12)));
            out->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            out->push_back((char)(0x80 | (cp & 0x3F)));
        } else {
            out->push_back((char)(0xF0 | (cp >> 18)));
            out->push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
            out->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            out->push_back((char)(0x80 | (cp & 0x3F)));
        }
    }
    bool hex4(uint32_t *v) {
        if (n - i < 4) return fail("short \\u escape");
        *v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = s[i++];
            *v <<= 4;
            if (c >= '0' && c <= '9') *v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') *v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') *v |= (uint32_t)(c - 'A' + 10);
            else return fail("bad \\u escape");
        }
        return true;
    }
    bool string(std::string *out) {
        if (i >= n || s[i] != '"') return fail("expected a string");
        ++i;
        out->clear();
        while (i < n) {
            const char c = s[i++];
            if (c == '"') return true;
            if ((unsigned char)c < 0x20) return fail("control character in string");
            if (c != '\\') {
                out->push_back(c);
                continue;
            }
            if (i >= n) break;
            const char e = s[i++];
            switch (e) {
                case '"': out->push_back('"'); break;
                case '\\': out->push_back('\\'); break;
                case '/': out->push_back('/'); break;
                case 'b': out->push_back('\b'); break;
                case 'f': out->push_back('\f'); break;
                case 'n': out->push_back('\n'); break;
                case 'r': out->push_back('\r'); break;
                case 't': out->push_back('\t'); break;
                case 'u': {
                    uint32_t cp;
                    if (!hex4(&cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00) {
                        uint32_t lo;
                        if (n - i < 2 || s[i] != '\\' || s[i + 1] != 'u') return fail("lone surrogate");
                        i += 2;
                        if (!hex4(&lo) || lo < 0xDC00 || lo >= 0xE000) return fail("bad surrogate pair");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp < 0xE000) {
                        return fail("lone surrogate");
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: return fail("bad escape");
            }
        }
        return fail("unterminated string");
    }
    bool number(Json *v) {
        const size_t start = i;
        if (i < n && s[i] == '-') ++i;
        if (i >= n) return fail("bad number");
        if (s[i] == '0') {
            ++i;
        } else if (s[i] >= '1' && s[i] <= '9') {
            while (i < n && s[i] >= '0' && s[i] <= '9') ++i;
        } else {
            return fail("bad number");
        }
        if (i < n && s[i] == '.') {
            ++i;
            if (i >= n || s[i] < '0' || s[i] > '9') return fail("bad fraction");
            while (i < n && s[i] >= '0' && s[i] <= '9') ++i;
        }
        if (i < n && (s[i] == 'e' || s[i] == 'E')) {
            ++i;
            if (i < n && (s[i] == '+' || s[i] == '-')) ++i;
            if (i >= n || s[i] < '0' || s[i] > '9') return fail("bad exponent");
            while (i < n && s[i] >= '0' && s[i] <= '9') ++i;
        }
        v->kind = Json::Number;
        v->text.assign(s + start, i - start);
        return true;
    }
    bool value(Json *v, int depth) {
        if (depth > 256) return fail("nesting too deep");
        space();
        if (i >= n) return fail("unexpected end");
        const char c = s[i];
        if (c == '{') {
            ++i;
            v->kind = Json::Object;
            space();
            if (i < n && s[i] == '}') {
                ++i;
                return true;
            }
            while (true) {
                space();
                std::string key;
                if (!string(&key)) return false;
                space();
                if (i >= n || s[i] != ':') return fail("expected ':'");
                ++i;
                v->fields.emplace_back(std::move(key), Json{});
                if (!value(&v->fields.back().second, depth + 1)) return false;
                space();
                if (i < n && s[i] == ',') {
                    ++i;
                    continue;
                }
                if (i < n && s[i] == '}') {
                    ++i;
                    return true;
                }
                return fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            ++i;
            v->kind = Json::Array;
            space();
            if (i < n && s[i] == ']') {
                ++i;
                return true;
            }
            while (true) {
                v->items.emplace_back();
                if (!value(&v->items.back(), depth + 1)) return false;
                space();
                if (i < n && s[i] == ',') {
                    ++i;
                    continue;
                }
                if (i < n && s[i] == ']') {
                    ++i;
                    return true;
                }
                return fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v->kind = Json::String;
            return string(&v->text);
        }
        if (c == 't') {
            v->kind = Json::Bool;
            v->boolean = true;
            return literal("true");
        }
        if (c == 'f') {
            v->kind = Json::Bool;
            v->boolean = false;
            return literal("false");
        }
        if (c == 'n') {
            v->kind = Json::Null;
            return literal("null");
        }
        return number(v);
    }
};

}  // namespace

bool parse_json(const char *s, size_t n, Json *out, std::string *error) {
    Reader r{s, n};
    *out = Json{};
    if (!r.value(out, 0)) {
        *error = r.error;
        return false;
    }
    r.space();
    if (r.i != n) {
        r.fail("trailing characters");
        *error = r.error;
        return false;
    }
    return true;
}

std::string json_quote(const std::string &s) {
    std::string out = "\"";
    for (unsigned char c : s) {
        switch (c) {
            case '"': out += "\\\""; break;
            case '\\': out += "\\\\"; break;
            case '\n': out += "\\n"; break;
            case '\r': out += "\\r"; break;
            case '\t': out += "\\t"; break;
            case '\b': out += "\\b"; break;
            case '\f': out += "\\f"; break;
            default:
                if (c < 0x20) {
                    char buf[8];
                    std::snprintf(buf, sizeof buf, "\\u%04x", c);
                    out += buf;
                } else {
                    out.push_back((char)c);
                }
        }
    }
    out += "\"";
    return out;
}

void write_json(const Json &v, std::string *out) {
    switch (v.kind) {
        case Json::Null: *out += "null"; break;
        case Json::Bool: *out += v.boolean ? "true" : "false"; break;
        case Json::Number: *out += v.text; break;
        case Json::String: *out += json_quote(v.text); break;
        case Json::Array:
            out->push_back('[');
            for (size_t k = 0; k < v.items.size(); ++k) {
                if (k) out->push_back(',');
                write_json(v.items[k], out);
            }
            out->push_back(']');
            break;
        case Json::Object:
            out->push_back('{');
            for (size_t k = 0; k < v.fields.size(); ++k) {
                if (k) out->push_back(',');
                *out += json_quote(v.fields[k].first);
                out->push_back(':');
                write_json(v.fields[k].second, out);
            }
            out->push_back('}');
            break;
    }
}

}  // namespace dag
}  // namespace chelis
