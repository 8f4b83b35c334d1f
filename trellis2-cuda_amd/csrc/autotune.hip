// Tile choices replayed from a FlexGEMM autotune cache file (host code only).
//
// The reference picks its masked implicit-GEMM tiles (B1 rows per schedule block, BK channels per K step, split
// factor S) from FlexGEMM's persisted autotune JSON (src/spconv.cu:176-221, assets/flexgemm_autotune.json); the
// schedule lists valid(B1) depend on B1. This build runs its own fixed tiles, so the table does not drive the
// kernels; `spconv_cfg_autotune` returns what the reference would pick, for callers that want the reference's
// schedule blocks (valid(B1)) or a like-for-like comparison.
//
// File layout used (per device name): two sections keyed by Python tuple strings,
//   <M>_splitk.<...>_splitk               "(2^L, Ci, Co, 27)"                 -> {"SPLITK": S}
//   <M>_splitk.<...>_splitk_kernel        "(L, Ci, Co, 27, S, True, ...)"     -> {"kwargs": {"B1", "BK", ...}}
//   <M>.<...>_kernel                      "(L, Ci, Co, 27, True, ...)"        -> same, S = 1 (read last, so it wins)
// with L = floor(log2 N). Missing entries give B1 = 128, BK = 64, S = 1, the reference's fallback.
#include <cstdlib>
#include <fstream>
#include <map>
#include <sstream>
#include <stdexcept>
#include <tuple>

#include "spconv.h"

namespace {
// A small JSON reader: objects keep their members in file order; arrays, literals and numbers are kept as text.
struct JNode {
  bool object = false;
  std::string text;  // string contents (unescaped) or the literal's text
  std::vector<std::pair<std::string, JNode>> members;
  const JNode* get(const std::string& k) const {
    for (const auto& m : members)
      if (m.first == k) return &m.second;
    return nullptr;
  }
};

struct JParser {
  const std::string& s;
  size_t i = 0;
  void ws() {
    while (i < s.size() && (s[i] == ' ' || s[i] == '\n' || s[i] == '\r' || s[i] == '\t')) i++;
  }
  [[noreturn]] void fail(const char* what) {
    throw std::runtime_error(std::string("autotune json: ") + what + " at byte " + std::to_string(i));
  }
  std::string str() {
    if (s[i] != '"') fail("expected a string");
    std::string out;
    for (i++; i < s.size() && s[i] != '"'; i++) {
      if (s[i] == '\\') {
        if (++i >= s.size()) break;
        const char c = s[i];
        out += c == 'n' ? '\n' : c == 't' ? '\t' : c;  // \uXXXX is not used by the cache files; kept verbatim
      } else {
        out += s[i];
      }
    }
    if (i >= s.size()) fail("unterminated string");
    i++;
    return out;
  }
  JNode value() {
    ws();
    if (i >= s.size()) fail("unexpected end");
    JNode n;
    if (s[i] == '{') {
      n.object = true;
      i++;
      ws();
      if (s[i] == '}') {
        i++;
        return n;
      }
      for (;;) {
        ws();
        std::string k = str();
        ws();
        if (s[i] != ':') fail("expected ':'");
        i++;
        n.members.emplace_back(std::move(k), value());
        ws();
        if (s[i] == ',') {
          i++;
          continue;
        }
        if (s[i] == '}') {
          i++;
          return n;
        }
        fail("expected ',' or '}'");
      }
    }
    if (s[i] == '[') {  // kept as text, nesting respected
      const size_t b = i;
      int depth = 0;
      for (; i < s.size(); i++) {
        if (s[i] == '"') {
          str();
          i--;
        } else if (s[i] == '[') {
          depth++;
        } else if (s[i] == ']' && --depth == 0) {
          i++;
          break;
        }
      }
      n.text = s.substr(b, i - b);
      return n;
    }
    if (s[i] == '"') {
      n.text = str();
      return n;
    }
    const size_t b = i;
    while (i < s.size() && s[i] != ',' && s[i] != '}' && s[i] != ']' && s[i] != ' ' && s[i] != '\n') i++;
    n.text = s.substr(b, i - b);
    return n;
  }
};

// "(a, b, c, ...)" -> {"a", "b", "c", ...}
std::vector<std::string> tuple_fields(const std::string& k) {
  std::vector<std::string> f;
  if (k.size() < 2 || k.front() != '(' || k.back() != ')') return f;
  std::string cur;
  for (size_t i = 1; i + 1 < k.size(); i++) {
    if (k[i] == ',') {
      f.push_back(cur);
      cur.clear();
      if (i + 1 < k.size() && k[i + 1] == ' ') i++;
    } else {
      cur += k[i];
    }
  }
  f.push_back(cur);
  return f;
}

bool to_int(const std::string& t, int& v) {
  if (t.empty()) return false;
  for (char c : t)
    if (c < '0' || c > '9') return false;
  v = std::stoi(t);
  return true;
}

struct Table {
  std::map<std::tuple<int, int, int>, int> split;                         // (L, Ci, Co) -> S
  std::map<std::tuple<int, int, int, int>, std::pair<int, int>> tiles;  // (L, Ci, Co, S) -> (B1, BK)
};

Table load_table(const std::string& path, const std::string& device) {
  std::ifstream f(path);
  REQ(f.good(), "cannot read the autotune cache %s", path.c_str());
  std::stringstream ss;
  ss << f.rdbuf();
  const std::string text = ss.str();
  JParser p{text};
  const JNode root = p.value();
  Table t;
  const JNode* dev = root.get(device);
  if (!dev) return t;  // no section for this device: every lookup falls back
  const std::string M = "flex_gemm.kernels.triton.spconv.sparse_submanifold_conv_fwd_masked_implicit_gemm";
  if (const JNode* sec = dev->get(M + "_splitk.sparse_submanifold_conv_fwd_masked_implicit_gemm_splitk"))
    for (const auto& m : sec->members) {
      const auto k = tuple_fields(m.first);
      int L, ci, co, s;
      const JNode* sk = m.second.get("SPLITK");
      if (k.size() == 4 && k[0].rfind("2^", 0) == 0 && to_int(k[0].substr(2), L) && to_int(k[1], ci) &&
          to_int(k[2], co) && k[3] == "27" && sk && to_int(sk->text, s))
        t.split[{L, ci, co}] = s;
    }
  for (const std::string& name : {M + "_splitk.sparse_submanifold_conv_fwd_masked_implicit_gemm_splitk_kernel",
                                   M + ".sparse_submanifold_conv_fwd_masked_implicit_gemm_kernel"}) {
    const JNode* sec = dev->get(name);
    if (!sec) continue;
    for (const auto& m : sec->members) {
      const auto k = tuple_fields(m.first);
      int L, ci, co, s = 1, b1, bk;
      if (k.size() < 5 || !to_int(k[0], L) || !to_int(k[1], ci) || !to_int(k[2], co) || k[3] != "27") continue;
      size_t at = 4;
      if (to_int(k[4], s)) at = 5;
      if (at >= k.size() || k[at] != "True") continue;
      const JNode* kw = m.second.get("kwargs");
      const JNode* jb1 = kw ? kw->get("B1") : nullptr;
      const JNode* jbk = kw ? kw->get("BK") : nullptr;
      if (jb1 && jbk && to_int(jb1->text, b1) && to_int(jbk->text, bk)) t.tiles[{L, ci, co, s}] = {b1, bk};
    }
  }
  return t;
}
}  // namespace

SpConvCfg spconv_cfg_autotune(const std::string& path, const std::string& device, i64 N, int Ci, int Co, bool strict) {
  static std::map<std::pair<std::string, std::string>, Table> cache;  // callers serialize (the C ABI holds a mutex)
  auto it = cache.find({path, device});
  if (it == cache.end()) it = cache.emplace(std::make_pair(path, device), load_table(path, device)).first;
  const Table& t = it->second;
  int L = 0;
  while (((i64)2 << L) <= N) L++;
  const auto si = t.split.find({L, Ci, Co});
  const int S = si == t.split.end() ? 1 : si->second;
  SpConvCfg c{128, 64, S};
  const auto ti = t.tiles.find({L, Ci, Co, S});
  if (ti != t.tiles.end()) {
    c.B1 = ti->second.first;
    c.BK = ti->second.second;
  } else {
    // strict replay: a miss is an error instead of the (128, 64, S) default, as the reference does under
    // T2_STRICT=1 (src/spconv.cu:219), so a replayed tile is never mistaken for a default one
    const char* e = getenv("T2_STRICT");
    REQ(!(strict || (e && std::string(e) == "1")), "no autotune entry for N=2^%d Ci=%d Co=%d S=%d", L, Ci, Co, S);
  }
  return c;
}
