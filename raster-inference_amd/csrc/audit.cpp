// Challenger-side comparison of checkpoint trace artifacts (host code only).
// Parsing follows ClaimedTrace::from_json_bytes / from_value
// (shared/api/audit.rs:34-82): the bytes must be one JSON value, that value
// an array, each element an object with exactly one key whose value is a
// string. Objects keep the last of repeated keys, as a JSON map does.
#include "audit.h"

#include <algorithm>
#include <cstdio>
#include <map>

namespace det_audit {

std::string json_quote(const std::string& v) {
  std::string o = "\"";
  for (unsigned char ch : v) {
    switch (ch) {
      case '"': o += "\\\""; break;
      case '\\': o += "\\\\"; break;
      case '\b': o += "\\b"; break;
      case '\f': o += "\\f"; break;
      case '\n': o += "\\n"; break;
      case '\r': o += "\\r"; break;
      case '\t': o += "\\t"; break;
      default:
        if (ch < 0x20) {
          char b[8];
          snprintf(b, sizeof b, "\\u%04x", unsigned(ch));
          o += b;
        } else {
          o += char(ch);
        }
    }
  }
  return o + "\"";
}

namespace {

// Maximum nesting of arrays and objects (a JSON reader's recursion limit).
constexpr int kMaxDepth = 127;

struct Value {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  std::string str;
  std::vector<Value> items;
  std::map<std::string, Value> members;
};

struct Reader {
  const unsigned char* p;
  const unsigned char* end;
  const unsigned char* begin;

  [[noreturn]] void fail(const std::string& what) const {
    throw Error("claimed trace artifact is not valid JSON: " + what + " at byte " + std::to_string(p - begin));
  }
  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool eat(char c) {
    if (p < end && *p == (unsigned char)c) {
      ++p;
      return true;
    }
    return false;
  }
  void literal(const char* word) {
    for (const char* w = word; *w; ++w)
      if (!eat(*w)) fail(std::string("expected `") + word + "`");
  }
  unsigned hex4() {
    unsigned v = 0;
    for (int i = 0; i < 4; ++i) {
      if (p >= end) fail("EOF in hex escape");
      const unsigned char c = *p++;
      unsigned d;
      if (c >= '0' && c <= '9') d = c - '0';
      else if (c >= 'a' && c <= 'f') d = c - 'a' + 10;
      else if (c >= 'A' && c <= 'F') d = c - 'A' + 10;
      else fail("invalid hex escape");
      v = v << 4 | d;
    }
    return v;
  }
  static void put_utf8(std::string& o, unsigned cp) {
    if (cp < 0x80) {
      o += char(cp);
    } else if (cp < 0x800) {
      o += char(0xC0 | cp >> 6);
      o += char(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      o += char(0xE0 | cp >> 12);
      o += char(0x80 | (cp >> 6 & 0x3F));
      o += char(0x80 | (cp & 0x3F));
    } else {
      o += char(0xF0 | cp >> 18);
      o += char(0x80 | (cp >> 12 & 0x3F));
      o += char(0x80 | (cp >> 6 & 0x3F));
      o += char(0x80 | (cp & 0x3F));
    }
  }
  // One well-formed UTF-8 sequence (no overlong forms, surrogates or code
  // points above U+10FFFF), copied to o.
  void utf8_seq(std::string& o) {
    const unsigned char c = *p;
    int n;
    unsigned lo = 0x80, hi = 0xBF;
    if (c >= 0xC2 && c <= 0xDF) n = 1;
    else if (c >= 0xE0 && c <= 0xEF) {
      n = 2;
      if (c == 0xE0) lo = 0xA0;
      if (c == 0xED) hi = 0x9F;
    } else if (c >= 0xF0 && c <= 0xF4) {
      n = 3;
      if (c == 0xF0) lo = 0x90;
      if (c == 0xF4) hi = 0x8F;
    } else {
      fail("invalid UTF-8 in string");
    }
    if (end - p <= n) fail("invalid UTF-8 in string");
    for (int i = 1; i <= n; ++i) {
      const unsigned char t = p[i];
      if (t < (i == 1 ? lo : 0x80u) || t > (i == 1 ? hi : 0xBFu)) fail("invalid UTF-8 in string");
    }
    o.append(reinterpret_cast<const char*>(p), size_t(n + 1));
    p += n + 1;
  }
  std::string string() {
    if (!eat('"')) fail("expected string");
    std::string o;
    for (;;) {
      if (p >= end) fail("EOF while parsing a string");
      const unsigned char c = *p;
      if (c == '"') {
        ++p;
        return o;
      }
      if (c < 0x20) fail("control character in string");
      if (c >= 0x80) {
        utf8_seq(o);
        continue;
      }
      ++p;
      if (c != '\\') {
        o += char(c);
        continue;
      }
      if (p >= end) fail("EOF while parsing a string");
      switch (*p++) {
        case '"': o += '"'; break;
        case '\\': o += '\\'; break;
        case '/': o += '/'; break;
        case 'b': o += '\b'; break;
        case 'f': o += '\f'; break;
        case 'n': o += '\n'; break;
        case 'r': o += '\r'; break;
        case 't': o += '\t'; break;
        case 'u': {
          unsigned cp = hex4();
          if (cp >= 0xDC00 && cp <= 0xDFFF) fail("lone trailing surrogate in hex escape");
          if (cp >= 0xD800 && cp <= 0xDBFF) {
            if (!(eat('\\') && eat('u'))) fail("lone leading surrogate in hex escape");
            const unsigned lo = hex4();
            if (lo < 0xDC00 || lo > 0xDFFF) fail("lone leading surrogate in hex escape");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          put_utf8(o, cp);
          break;
        }
        default:
          fail("invalid escape");
      }
    }
  }
  void digits() {
    if (p >= end || *p < '0' || *p > '9') fail("invalid number");
    while (p < end && *p >= '0' && *p <= '9') ++p;
  }
  void number() {
    eat('-');
    if (eat('0')) {
      if (p < end && *p >= '0' && *p <= '9') fail("invalid number");
    } else {
      digits();
    }
    if (eat('.')) digits();
    if (p < end && (*p == 'e' || *p == 'E')) {
      ++p;
      if (!eat('+')) eat('-');
      digits();
    }
  }
  Value value(int depth) {
    ws();
    if (p >= end) fail("EOF while parsing a value");
    Value v;
    const unsigned char c = *p;
    if (c == '[' || c == '{') {
      if (depth >= kMaxDepth) fail("recursion limit exceeded");
      ++p;
      const char close = c == '[' ? ']' : '}';
      v.kind = c == '[' ? Value::Array : Value::Object;
      ws();
      if (eat(close)) return v;
      for (;;) {
        if (v.kind == Value::Array) {
          v.items.push_back(value(depth + 1));
        } else {
          ws();
          std::string key = string();
          ws();
          if (!eat(':')) fail("expected `:`");
          v.members[std::move(key)] = value(depth + 1);
        }
        ws();
        if (eat(close)) return v;
        if (!eat(',')) fail(std::string("expected `,` or `") + close + "`");
      }
    }
    if (c == '"') {
      v.kind = Value::String;
      v.str = string();
    } else if (c == 't') {
      literal("true");
      v.kind = Value::Bool;
    } else if (c == 'f') {
      literal("false");
      v.kind = Value::Bool;
    } else if (c == 'n') {
      literal("null");
    } else if (c == '-' || (c >= '0' && c <= '9')) {
      number();
      v.kind = Value::Number;
    } else {
      fail("expected value");
    }
    return v;
  }
};

}  // namespace

std::vector<Entry> parse_trace(const char* bytes, size_t n) {
  const auto* b = reinterpret_cast<const unsigned char*>(bytes);
  Reader r{b, b + n, b};
  Value doc = r.value(0);
  r.ws();
  if (r.p != r.end) r.fail("trailing characters");
  if (doc.kind != Value::Array) throw Error("claimed trace artifact should be a JSON array of checkpoint entries");
  std::vector<Entry> out;
  std::map<std::string, uint64_t> seen;
  for (size_t i = 0; i < doc.items.size(); ++i) {
    const Value& e = doc.items[i];
    const std::string at = "claimed trace entry " + std::to_string(i);
    if (e.kind != Value::Object) throw Error(at + " should be an object");
    if (e.members.size() != 1) throw Error(at + " should contain exactly one commitment");
    const auto& kv = *e.members.begin();
    if (kv.second.kind != Value::String) throw Error(at + " commitment should be a string");
    out.push_back({i, kv.first, ++seen[kv.first], kv.second.str});
  }
  return out;
}

// locate_first_divergence (runtime/roles/challenger.rs:136-183)
bool first_divergence(const std::vector<Entry>& claimed, const std::vector<Entry>& replayed, Divergence* out) {
  Divergence d;
  const size_t common = std::min(claimed.size(), replayed.size());
  for (size_t i = 0; i < common; ++i) {
    const Entry& c = claimed[i];
    const Entry& r = replayed[i];
    if (c.checkpoint_id == r.checkpoint_id && c.commitment == r.commitment) continue;
    d.entry_index = i;
    d.checkpoint_id = r.checkpoint_id;
    d.occurrence = r.occurrence;
    if (c.checkpoint_id != r.checkpoint_id) {
      d.has_claimed_checkpoint_id = true;
      d.claimed_checkpoint_id = c.checkpoint_id;
    }
    d.has_claimed_commitment = d.has_replayed_commitment = true;
    d.claimed_commitment = c.commitment;
    d.replayed_commitment = r.commitment;
    *out = d;
    return true;
  }
  if (claimed.size() == replayed.size()) return false;
  // length divergence: the first unmatched entry of the longer sequence
  const bool replay_longer = replayed.size() > common;
  const Entry& e = replay_longer ? replayed[common] : claimed[common];
  d.entry_index = common;
  d.checkpoint_id = e.checkpoint_id;
  d.occurrence = e.occurrence;
  (replay_longer ? d.has_replayed_commitment : d.has_claimed_commitment) = true;
  (replay_longer ? d.replayed_commitment : d.claimed_commitment) = e.commitment;
  *out = d;
  return true;
}

// detour_spec_for (challenger.rs:185-210) with DETOURABLE_ROUTINES
// (challenger.rs:28-37) and RasterDetourSpec's Display (checkpoints.rs:163-171).
std::string detour_spec(const Divergence& d) {
  static const char* const kDetourable[] = {
      "input.embedding",     "prefill.prepare_aux", "prefill.range",              "prefill.finalize",
      "decode.select_token", "decode.layer_range",  "decode.transition_finalize", "output.finalize"};
  if (d.has_claimed_checkpoint_id || !d.has_claimed_commitment || !d.has_replayed_commitment) return "";
  for (const char* id : kDetourable)
    if (d.checkpoint_id == id)
      return d.occurrence == 1 ? d.checkpoint_id : d.checkpoint_id + ":" + std::to_string(d.occurrence);
  return "";
}

std::string outcome_json(const std::vector<Entry>& claimed, const std::vector<Entry>& replayed, bool* diverged) {
  Divergence d;
  const bool div = first_divergence(claimed, replayed, &d);
  if (diverged) *diverged = div;
  if (!div) return "{\"diverged\":false}";
  std::string o = "{\"diverged\":true,\"divergence\":{\"entry_index\":" + std::to_string(d.entry_index) +
                  ",\"checkpoint_id\":" + json_quote(d.checkpoint_id) +
                  ",\"occurrence\":" + std::to_string(d.occurrence);
  if (d.has_claimed_checkpoint_id) o += ",\"claimed_checkpoint_id\":" + json_quote(d.claimed_checkpoint_id);
  if (d.has_claimed_commitment) o += ",\"claimed_commitment\":" + json_quote(d.claimed_commitment);
  if (d.has_replayed_commitment) o += ",\"replayed_commitment\":" + json_quote(d.replayed_commitment);
  const std::string spec = detour_spec(d);
  o += "},\"detour\":" + (spec.empty() ? std::string("null") : json_quote(spec)) + "}";
  return o;
}

std::vector<Entry> entries_of(const std::vector<std::pair<std::string, std::string>>& committed) {
  std::vector<Entry> out;
  std::map<std::string, uint64_t> seen;
  for (size_t i = 0; i < committed.size(); ++i)
    out.push_back({i, committed[i].first, ++seen[committed[i].first], committed[i].second});
  return out;
}

}  // namespace det_audit
