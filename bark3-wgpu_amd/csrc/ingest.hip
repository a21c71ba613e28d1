// Safetensors checkpoint reading on the host: the layout TensorReader reads
// (src/weights_io.rs:46-127) — an 8-byte little-endian header length, a JSON
// header {name: {"dtype", "shape", "data_offsets": [begin, end]}, "__metadata__":
// {...}}, then the tensor bytes (offsets relative to the end of the header) —
// and the sharded form, model.safetensors.index.json {"weight_map": {name:
// shard file}}. Only the header is parsed here; tensors are read one at a time
// by the caller.
#include <cstdio>
#include <map>
#include <set>
#include <string>
#include <sys/stat.h>
#include <vector>

#include "kernels.h"

namespace bark {
namespace {

// A small JSON reader for these two headers: objects, arrays, strings,
// numbers, true / false / null. Values are kept as a tree of nodes.
struct Json {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  double num = 0;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;
  const Json* get(const std::string& k) const {
    for (const auto& kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

struct JsonParser {
  const std::string& s;
  size_t i = 0;
  std::string where;
  [[noreturn]] void fail(const char* what) {
    throw Error{where + ": malformed JSON header (" + what + " at byte " + std::to_string(i) + ")"};
  }
  void ws() {
    while (i < s.size() && (s[i] == ' ' || s[i] == '\n' || s[i] == '\r' || s[i] == '\t')) ++i;
  }
  bool eat(char c) {
    ws();
    if (i < s.size() && s[i] == c) {
      ++i;
      return true;
    }
    return false;
  }
  std::string string() {
    ws();
    if (i >= s.size() || s[i] != '"') fail("expected a string");
    ++i;
    std::string out;
    while (true) {
      if (i >= s.size()) fail("unterminated string");
      const char c = s[i++];
      if (c == '"') break;
      if (c != '\\') {
        out += c;
        continue;
      }
      if (i >= s.size()) fail("unterminated escape");
      const char e = s[i++];
      switch (e) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {  // code point as UTF-8 (surrogate pairs joined)
          auto hex4 = [&]() {
            if (i + 4 > s.size()) fail("short \\u escape");
            unsigned v = 0;
            for (int k = 0; k < 4; ++k) {
              const char h = s[i++];
              v <<= 4;
              if (h >= '0' && h <= '9') v |= h - '0';
              else if (h >= 'a' && h <= 'f') v |= h - 'a' + 10;
              else if (h >= 'A' && h <= 'F') v |= h - 'A' + 10;
              else fail("bad \\u escape");
            }
            return v;
          };
          unsigned cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00 && i + 1 < s.size() && s[i] == '\\' && s[i + 1] == 'u') {
            i += 2;
            const unsigned lo = hex4();
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          if (cp < 0x80) {
            out += (char)cp;
          } else if (cp < 0x800) {
            out += (char)(0xC0 | (cp >> 6));
            out += (char)(0x80 | (cp & 0x3F));
          } else if (cp < 0x10000) {
            out += (char)(0xE0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
          } else {
            out += (char)(0xF0 | (cp >> 18));
            out += (char)(0x80 | ((cp >> 12) & 0x3F));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
          }
          break;
        }
        default: fail("bad escape");
      }
    }
    return out;
  }
  Json value(int depth = 0) {
    if (depth > 64) fail("nesting too deep");
    ws();
    if (i >= s.size()) fail("unexpected end");
    Json v;
    const char c = s[i];
    if (c == '{') {
      ++i;
      v.kind = Json::OBJ;
      if (eat('}')) return v;
      do {
        std::string k = string();
        if (!eat(':')) fail("expected ':'");
        v.obj.emplace_back(std::move(k), value(depth + 1));
      } while (eat(','));
      if (!eat('}')) fail("expected '}'");
    } else if (c == '[') {
      ++i;
      v.kind = Json::ARR;
      if (eat(']')) return v;
      do v.arr.push_back(value(depth + 1));
      while (eat(','));
      if (!eat(']')) fail("expected ']'");
    } else if (c == '"') {
      v.kind = Json::STR;
      v.str = string();
    } else if (s.compare(i, 4, "true") == 0 || s.compare(i, 5, "false") == 0) {
      v.kind = Json::BOOL;
      v.num = s[i] == 't';
      i += s[i] == 't' ? 4 : 5;
    } else if (s.compare(i, 4, "null") == 0) {
      i += 4;
    } else {
      const size_t b = i;
      while (i < s.size() && (isdigit((unsigned char)s[i]) || s[i] == '-' || s[i] == '+' || s[i] == '.' ||
                              s[i] == 'e' || s[i] == 'E'))
        ++i;
      if (i == b) fail("unexpected character");
      v.kind = Json::NUM;
      v.num = std::stod(s.substr(b, i - b));
    }
    return v;
  }
};

Json parse_json(const std::string& text, const std::string& where) {
  JsonParser p{text, 0, where};
  Json v = p.value();
  p.ws();
  if (p.i != text.size()) p.fail("trailing data");
  return v;
}

bool is_dir(const std::string& p) {
  struct stat st;
  return stat(p.c_str(), &st) == 0 && S_ISDIR(st.st_mode);
}

bool exists(const std::string& p) {
  struct stat st;
  return stat(p.c_str(), &st) == 0;
}

std::string read_text(const std::string& path) {
  FILE* f = std::fopen(path.c_str(), "rb");
  BARK_REQUIRE(f, "cannot open " + path);
  std::string out;
  char buf[1 << 16];
  size_t n;
  while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) out.append(buf, n);
  std::fclose(f);
  return out;
}

// A non-negative integer below 2^53 (every such integer is exact in the
// double the parser holds; larger values are rejected before any cast).
int64_t as_int(const Json& v, const std::string& where) {
  BARK_REQUIRE(v.kind == Json::NUM && v.num >= 0 && v.num < 9007199254740992.0 &&
                   v.num == (double)(int64_t)v.num,
               where + ": expected an integer below 2^53");
  return (int64_t)v.num;
}

}  // namespace

int64_t shape_elements(const std::vector<int64_t>& shape, const std::string& where) {
  int64_t n = 1;
  for (int64_t d : shape)
    BARK_REQUIRE(!__builtin_mul_overflow(n, d, &n) && n < (int64_t(1) << 53),
                 where + ": element count of the shape overflows");
  return n;
}

std::vector<std::string> safetensors_files(const std::string& path) {
  if (!is_dir(path)) {
    BARK_REQUIRE(exists(path), "no such checkpoint: " + path);
    return {path};
  }
  const std::string index = path + "/model.safetensors.index.json";
  if (!exists(index)) return {path + "/model.safetensors"};
  const Json idx = parse_json(read_text(index), index);
  const Json* map = idx.get("weight_map");
  BARK_REQUIRE(map && map->kind == Json::OBJ, index + ": no weight_map object");
  std::set<std::string> shards;  // sorted, each once (src/weights_io.rs:53-62)
  for (const auto& kv : map->obj) {
    BARK_REQUIRE(kv.second.kind == Json::STR, index + ": weight_map values must be file names");
    BARK_REQUIRE(kv.second.str.find('/') == std::string::npos, index + ": shard names must be plain file names");
    shards.insert(kv.second.str);
  }
  std::vector<std::string> out;
  for (const auto& s : shards) out.push_back(path + "/" + s);
  return out;
}

std::vector<StTensor> safetensors_header(const std::string& file) {
  FILE* f = std::fopen(file.c_str(), "rb");
  BARK_REQUIRE(f, "cannot open " + file);
  unsigned char len8[8];
  const bool got = std::fread(len8, 1, 8, f) == 8;
  uint64_t hlen = 0;
  for (int k = 7; k >= 0; --k) hlen = (hlen << 8) | len8[k];
  std::fseek(f, 0, SEEK_END);
  const uint64_t size = (uint64_t)std::ftell(f);
  if (!got || hlen > size - 8 || hlen > (1ull << 30)) {
    std::fclose(f);
    throw Error{file + ": not a safetensors file (header length)"};
  }
  std::string header(hlen, '\0');
  std::fseek(f, 8, SEEK_SET);
  const bool ok = std::fread(&header[0], 1, hlen, f) == hlen;
  std::fclose(f);
  BARK_REQUIRE(ok, file + ": short read of the header");
  const Json h = parse_json(header, file);
  BARK_REQUIRE(h.kind == Json::OBJ, file + ": header is not an object");
  const uint64_t data = 8 + hlen, avail = size - data;
  std::vector<StTensor> out;
  for (const auto& kv : h.obj) {
    if (kv.first == "__metadata__") continue;
    const std::string where = file + ": " + kv.first;
    const Json& e = kv.second;
    const Json *dt = e.get("dtype"), *sh = e.get("shape"), *off = e.get("data_offsets");
    BARK_REQUIRE(e.kind == Json::OBJ && dt && dt->kind == Json::STR && sh && sh->kind == Json::ARR && off &&
                     off->kind == Json::ARR && off->arr.size() == 2,
                 where + ": malformed tensor entry");
    StTensor t;
    t.name = kv.first;
    t.dtype = dt->str;
    for (const auto& d : sh->arr) t.shape.push_back(as_int(d, where));
    t.numel = shape_elements(t.shape, where);
    t.begin = data + (uint64_t)as_int(off->arr[0], where);
    t.end = data + (uint64_t)as_int(off->arr[1], where);
    BARK_REQUIRE(t.begin <= t.end && t.end - data <= avail, where + ": data outside the file");
    out.push_back(std::move(t));
  }
  return out;
}

// probe (src/weights_io.rs:208-297): what a checkpoint holds, from its
// header(s) alone, as a JSON object {release, layout, tensors, weights,
// layers, hidden, ffn, vocab}. A 4-bit code word (U32) counts as eight
// weights; per-row level tables (".levels") are not weights.
std::string safetensors_probe(const std::string& path) {
  const std::string dir = is_dir(path) ? path : "";
  std::map<std::string, StTensor> entries;
  for (const std::string& f : safetensors_files(path))
    for (StTensor& t : safetensors_header(f)) entries[t.name] = std::move(t);
  bool lowbit = false;
  std::set<std::string> dtypes;
  uint64_t weights = 0;
  for (const auto& kv : entries) {
    const std::string& name = kv.first;
    if (name.size() >= 7 && name.compare(name.size() - 7, 7, ".levels") == 0) continue;
    const std::string& dt = kv.second.dtype;
    if (dt != "BF16" && dt != "F16" && dt != "F32" && dt != "U32") continue;  // never read
    dtypes.insert(dt);
    uint64_t n = (uint64_t)kv.second.numel;
    if (dt == "U32") {
      lowbit = true;
      n *= 8;
    }
    weights += n;
  }
  const bool lowbit_json = !dir.empty() && exists(dir + "/lowbit.json");
  BARK_REQUIRE(!dtypes.count("U32") || lowbit_json || dir.empty(),
               path + ": weights are stored as 4-bit codes but lowbit.json is missing");
  lowbit = lowbit || lowbit_json;
  const char* layout = lowbit ? "low-bit" : dtypes.count("BF16") ? "bf16" : dtypes.count("F16") ? "f16"
                                                                            : dtypes.count("F32") ? "f32"
                                                                                                  : nullptr;
  BARK_REQUIRE(layout, path + ": no float or code tensors found");
  auto ffn_w = entries.find("encoder.layers.0.feed_forward1.linear1.weight");
  BARK_REQUIRE(ffn_w != entries.end() && ffn_w->second.shape.size() >= 2,
               path + ": not a Parakeet TDT checkpoint (no feed_forward1)");
  const int64_t ffn = ffn_w->second.shape[0];
  const int64_t hidden = lowbit ? ffn_w->second.shape[1] * 8 : ffn_w->second.shape[1];
  auto emb = entries.find("decoder.embedding.weight");
  const int64_t vocab = emb != entries.end() && !emb->second.shape.empty() ? emb->second.shape[0] : 0;
  std::set<long> layers;
  const std::string pre = "encoder.layers.";
  for (const auto& kv : entries) {
    if (kv.first.compare(0, pre.size(), pre) != 0) continue;
    const size_t dot = kv.first.find('.', pre.size());
    if (dot == std::string::npos || dot == pre.size()) continue;
    const std::string n = kv.first.substr(pre.size(), dot - pre.size());
    if (n.find_first_not_of("0123456789") == std::string::npos && n.size() < 10) layers.insert(std::stol(n));
  }
  std::string release = "null";
  if (!dir.empty() && exists(dir + "/bark3.json")) {
    try {
      const Json v = parse_json(read_text(dir + "/bark3.json"), dir + "/bark3.json");
      const Json* src = v.get("source");
      if (src && src->kind == Json::STR) {
        release = "\"";
        for (char ch : src->str) {  // JSON string escape
          if (ch == '"' || ch == '\\') release += '\\', release += ch;
          else if ((unsigned char)ch < 0x20) {
            char b[8];
            snprintf(b, sizeof b, "\\u%04x", ch);
            release += b;
          } else release += ch;
        }
        release += "\"";
      }
    } catch (const Error&) {
      // an unreadable bark3.json names no release, as in the reference
    }
  }
  char buf[384];
  snprintf(buf, sizeof buf,
           ",\"layout\":\"%s\",\"tensors\":%zu,\"weights\":%llu,\"layers\":%zu,\"hidden\":%lld,"
           "\"ffn\":%lld,\"vocab\":%lld}",
           layout, entries.size(), (unsigned long long)weights, layers.size(), (long long)hidden, (long long)ffn,
           (long long)vocab);
  return "{\"release\":" + release + buf;
}

void safetensors_read(const std::string& file, const StTensor& t, void* dst) {
  FILE* f = std::fopen(file.c_str(), "rb");
  BARK_REQUIRE(f, "cannot open " + file);
  const size_t n = (size_t)(t.end - t.begin);
  const bool ok = std::fseek(f, (long)t.begin, SEEK_SET) == 0 && std::fread(dst, 1, n, f) == n;
  std::fclose(f);
  BARK_REQUIRE(ok, file + ": short read of " + t.name);
}

}  // namespace bark
