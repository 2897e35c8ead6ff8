// The wire parser (graph text -> Graph) and the fusion plan.
//
// The parser validates what the OCaml type system guarantees upstream
// (operand dtypes, operator/dtype combinations, shapes), so a malformed
// graph is an Invalid_argument at compile time rather than a bad kernel.

#include <cstdlib>
#include <cstring>
#include <sstream>
#include <unordered_map>

#include "internal.hpp"

namespace cchip {

int64_t row_length(const std::vector<int64_t> &shape) { return shape.empty() ? 1 : shape.back(); }

namespace {

struct Lexer {
  const char *p;
  int line = 1;
  bool eol() {
    while (*p == ' ' || *p == '\t' || *p == '\r') p++;
    return *p == '\n' || *p == 0;
  }
  void next_line() {
    while (*p && *p != '\n') p++;
    if (*p == '\n') {
      p++;
      line++;
    }
  }
  std::string tok() {
    if (eol()) throw InvalidArgument(strf("graph wire line %d: missing field", line));
    const char *s = p;
    while (*p && *p != ' ' && *p != '\t' && *p != '\n' && *p != '\r') p++;
    return std::string(s, p - s);
  }
  int64_t integer() {
    std::string t = tok();
    char *end = nullptr;
    long long v = strtoll(t.c_str(), &end, 10);
    if (*end || t.empty()) throw InvalidArgument(strf("graph wire line %d: bad integer '%s'", line, t.c_str()));
    return v;
  }
};

DT parse_dt(Lexer &lx) {
  std::string t = lx.tok();
  if (t == "f32") return DT::F32;
  if (t == "f64") return DT::F64;
  if (t == "i32") return DT::I32;
  if (t == "i64") return DT::I64;
  if (t == "bool") return DT::BOOL;
  throw InvalidArgument(strf("graph wire line %d: bad dtype '%s'", lx.line, t.c_str()));
}

std::string unescape(const std::string &t) {
  if (t == "%") return "";
  std::string o;
  for (size_t i = 0; i < t.size(); i++) {
    if (t[i] == '%' && i + 2 < t.size()) {
      char hx[3] = {t[i + 1], t[i + 2], 0};
      o.push_back((char)strtol(hx, nullptr, 16));
      i += 2;
    } else {
      o.push_back(t[i]);
    }
  }
  return o;
}

int find_op(const std::string &t, const char *const *names, int n, int line) {
  for (int i = 0; i < n; i++)
    if (t == names[i]) return i;
  throw InvalidArgument(strf("graph wire line %d: bad operator '%s'", line, t.c_str()));
}

const char *const kBin[] = {"add", "sub", "mul", "div", "min", "max", "and", "or", "xor", "shl", "shr"};
const char *const kUn[] = {"neg", "sqrt", "exp", "log", "abs", "sin", "cos", "erf", "erfinv"};
const char *const kCmp[] = {"eq", "ne", "lt", "le", "gt", "ge"};
const char *const kLogic[] = {"and", "or"};

}  // namespace

Graph parse_wire(const std::string &text) {
  Graph g;
  Lexer lx{text.c_str()};
  std::unordered_map<int64_t, int> xpos, tpos;
  if (lx.tok() != "cchip-graph") throw InvalidArgument("graph wire: not a cchip-graph text");
  if (lx.integer() != 1) throw InvalidArgument("graph wire: unsupported version");
  g.name = unescape(lx.tok());
  lx.next_line();
  auto xref = [&](Lexer &l) {
    int64_t id = l.integer();
    auto it = xpos.find(id);
    if (it == xpos.end()) throw InvalidArgument(strf("graph wire line %d: unknown expression %lld", l.line, (long long)id));
    return it->second;
  };
  auto tref = [&](Lexer &l) {
    int64_t id = l.integer();
    auto it = tpos.find(id);
    if (it == tpos.end()) throw InvalidArgument(strf("graph wire line %d: unknown tensor %lld", l.line, (long long)id));
    return it->second;
  };
  bool ended = false;
  while (*lx.p) {
    if (lx.eol()) {
      lx.next_line();
      continue;
    }
    std::string tag = lx.tok();
    if (tag == "x") {
      XNode x;
      x.id = lx.integer();
      std::string kind = lx.tok();
      x.dt = parse_dt(lx);
      int L = lx.line;
      auto need = [&](bool ok, const char *what) {
        if (!ok) throw InvalidArgument(strf("graph wire line %d: %s", L, what));
      };
      if (kind == "const") {
        x.kind = XK::Const;
        std::string t = lx.tok();
        if (dt_is_float(x.dt)) {
          uint64_t bits = strtoull(t.c_str(), nullptr, 16);
          memcpy(&x.f, &bits, 8);
        } else {
          x.i = strtoll(t.c_str(), nullptr, 10);
        }
      } else if (kind == "arg") {
        x.kind = XK::Arg;
        x.arg = (int)lx.integer();
        need(x.arg == 0 || x.arg == 1, "Arg index must be 0 or 1");
      } else if (kind == "index") {
        x.kind = XK::Index;
        need(x.dt == DT::I32, "Index is i32");
      } else if (kind == "bin") {
        x.kind = XK::Bin;
        x.op = find_op(lx.tok(), kBin, 11, L);
        x.a = xref(lx);
        x.b = xref(lx);
        need(g.xs[x.a].dt == x.dt && g.xs[x.b].dt == x.dt, "binop operand dtype mismatch");
        need(x.dt != DT::BOOL, "binop on bool");
        need(!(dt_is_float(x.dt) && x.op >= B_AND), "bitwise operator or shift on a float dtype");
      } else if (kind == "un") {
        x.kind = XK::Un;
        x.op = find_op(lx.tok(), kUn, 9, L);
        x.a = xref(lx);
        need(g.xs[x.a].dt == x.dt, "unop operand dtype mismatch");
        need(x.dt != DT::BOOL, "unop on bool");
        need(dt_is_float(x.dt) || x.op == U_NEG || x.op == U_ABS, "float-only unop on an integer dtype");
      } else if (kind == "cmp") {
        x.kind = XK::Cmp;
        x.op = find_op(lx.tok(), kCmp, 6, L);
        x.a = xref(lx);
        x.b = xref(lx);
        need(x.dt == DT::BOOL, "comparison has dtype bool");
        need(g.xs[x.a].dt == g.xs[x.b].dt, "comparison operand dtype mismatch");
      } else if (kind == "logic") {
        x.kind = XK::Logic;
        x.op = find_op(lx.tok(), kLogic, 2, L);
        x.a = xref(lx);
        x.b = xref(lx);
        need(x.dt == DT::BOOL && g.xs[x.a].dt == DT::BOOL && g.xs[x.b].dt == DT::BOOL, "logic is on bool");
      } else if (kind == "not") {
        x.kind = XK::Not;
        x.a = xref(lx);
        need(x.dt == DT::BOOL && g.xs[x.a].dt == DT::BOOL, "not is on bool");
      } else if (kind == "select") {
        x.kind = XK::Select;
        x.a = xref(lx);
        x.b = xref(lx);
        x.c = xref(lx);
        need(g.xs[x.a].dt == DT::BOOL, "select condition must be bool");
        need(g.xs[x.b].dt == x.dt && g.xs[x.c].dt == x.dt, "select branch dtype mismatch");
      } else if (kind == "cast") {
        x.kind = XK::Cast;
        x.a = xref(lx);
      } else {
        throw InvalidArgument(strf("graph wire line %d: bad expression kind '%s'", L, kind.c_str()));
      }
      if (!xpos.emplace(x.id, (int)g.xs.size()).second)
        throw InvalidArgument(strf("graph wire line %d: duplicate expression id", L));
      g.xs.push_back(x);
    } else if (tag == "t") {
      TNode t;
      t.id = lx.integer();
      std::string kind = lx.tok();
      t.dt = parse_dt(lx);
      int L = lx.line;
      auto need = [&](bool ok, const char *what) {
        if (!ok) throw InvalidArgument(strf("graph wire line %d: %s", L, what));
      };
      int64_t rank = lx.integer();
      need(rank >= 0 && rank <= 8, "rank must be 0..8");
      // Element counts and every extent stay below 2^31 (device indexes
      // are 32-bit, lower.ml:27-31); the product is checked before each
      // multiplication, so no extent list can wrap it.
      const int64_t kMaxNumel = (int64_t(1) << 31) - 1;
      t.numel = 1;
      for (int64_t i = 0; i < rank; i++) {
        int64_t d = lx.integer();
        need(d >= 0, "negative extent");
        need(d <= kMaxNumel, "more than 2^31-1 elements in one tensor");
        need(d == 0 || t.numel <= kMaxNumel / d, "more than 2^31-1 elements in one tensor");
        t.shape.push_back(d);
        t.numel *= d;
      }
      need(t.dt != DT::BOOL, "bool tensors are not storable");
      auto body_dt = [&](int x) { return g.xs[x].dt; };
      if (kind == "param") {
        t.kind = TK::Param;
        t.pname = unescape(lx.tok());
      } else if (kind == "iota") {
        t.kind = TK::Iota;
        need(t.dt == DT::I32, "iota is i32");
      } else if (kind == "map") {
        t.kind = TK::Map;
        t.a = tref(lx);
        t.body = xref(lx);
        need(body_dt(t.body) == t.dt, "map body dtype mismatch");
        need(g.ts[t.a].shape == t.shape, "map shape mismatch");
      } else if (kind == "map2") {
        t.kind = TK::Map2;
        t.a = tref(lx);
        t.b = tref(lx);
        t.body = xref(lx);
        need(body_dt(t.body) == t.dt, "map2 body dtype mismatch");
        need(g.ts[t.a].shape == t.shape && g.ts[t.b].shape == t.shape, "map2 shape mismatch");
      } else if (kind == "reduce" || kind == "scan") {
        t.kind = kind == "reduce" ? TK::Reduce : TK::Scan;
        t.a = tref(lx);
        t.init = xref(lx);
        t.body = xref(lx);
        const TNode &s = g.ts[t.a];
        need(s.dt == t.dt && body_dt(t.body) == t.dt && body_dt(t.init) == t.dt, "reduce/scan dtype mismatch");
        need(!s.shape.empty(), "reduce/scan source must have rank >= 1");
        if (t.kind == TK::Reduce) {
          std::vector<int64_t> want(s.shape.begin(), s.shape.end() - 1);
          need(want == t.shape, "reduce output shape must drop the last axis");
        } else {
          need(s.shape == t.shape, "scan shape mismatch");
        }
      } else if (kind == "gather") {
        t.kind = TK::Gather;
        t.a = tref(lx);
        t.b = tref(lx);
        need(g.ts[t.a].dt == DT::I32, "gather index must be i32");
        need(g.ts[t.b].dt == t.dt && g.ts[t.a].shape == t.shape, "gather dtype/shape mismatch");
      } else if (kind == "scatter_add") {
        t.kind = TK::Scatter;
        t.a = tref(lx);
        t.b = tref(lx);
        need(g.ts[t.a].dt == DT::I32, "scatter_add index must be i32");
        need(g.ts[t.a].shape == g.ts[t.b].shape, "scatter_add idx/src shape mismatch");
        need(g.ts[t.b].dt == t.dt && (t.dt == DT::F32 || t.dt == DT::F64 || t.dt == DT::I32),
             "scatter_add dtype cannot be accumulated");
      } else if (kind == "matmul") {
        t.kind = TK::Matmul;
        t.a = tref(lx);
        t.b = tref(lx);
        const TNode &A = g.ts[t.a], &B = g.ts[t.b];
        need(A.shape.size() == 2 && B.shape.size() == 2 && A.shape[1] == B.shape[0] && t.shape.size() == 2 &&
                 t.shape[0] == A.shape[0] && t.shape[1] == B.shape[1],
             "matmul needs [m;k] x [k;n]");
        need(A.dt == t.dt && B.dt == t.dt, "matmul dtype mismatch");
      } else if (kind == "reshape") {
        t.kind = TK::Reshape;
        t.a = tref(lx);
        need(g.ts[t.a].numel == t.numel && g.ts[t.a].dt == t.dt, "reshape numel mismatch");
      } else if (kind == "broadcast") {
        t.kind = TK::Broadcast;
        t.a = tref(lx);
        need(g.ts[t.a].numel == 1 && g.ts[t.a].dt == t.dt, "broadcast source must have exactly one element");
      } else {
        throw InvalidArgument(strf("graph wire line %d: bad tensor kind '%s'", L, kind.c_str()));
      }
      if (!tpos.emplace(t.id, (int)g.ts.size()).second)
        throw InvalidArgument(strf("graph wire line %d: duplicate tensor id", L));
      g.ts.push_back(t);
    } else if (tag == "o") {
      std::string n = unescape(lx.tok());
      int p = tref(lx);
      for (auto &o : g.outputs)
        if (o.first == n) throw InvalidArgument("Graph.create: duplicate output name " + n);
      g.outputs.emplace_back(n, p);
    } else if (tag == "end") {
      ended = true;
      break;
    } else {
      throw InvalidArgument(strf("graph wire line %d: bad tag '%s'", lx.line, tag.c_str()));
    }
    if (!lx.eol()) throw InvalidArgument(strf("graph wire line %d: trailing fields", lx.line));
    lx.next_line();
  }
  if (!ended) throw InvalidArgument("graph wire: missing 'end'");
  if (g.outputs.empty()) throw InvalidArgument("Graph.create: a graph needs at least one output");
  // Param names are unique per node (graph.ml:278-291).
  std::map<std::string, int> seen;
  for (size_t i = 0; i < g.ts.size(); i++)
    if (g.ts[i].kind == TK::Param) {
      auto it = seen.find(g.ts[i].pname);
      if (it != seen.end()) throw InvalidArgument("Graph.create: two Param nodes named " + g.ts[i].pname);
      seen[g.ts[i].pname] = (int)i;
    }
  // Fan-out counts uses (edges), not distinct consumers (graph.ml:263-276).
  g.fan_out.assign(g.ts.size(), 0);
  for (auto &t : g.ts)
    for (int d : t.deps()) g.fan_out[d]++;
  return g;
}

// Dsl.transpose (dsl.ml:167-182) builds, for x : [m; n], the gather
// out[k] = x[(k - (k/m)*m) * n + k/m] over iota [n; m]. Recognising that
// exact shape lets the backend drop the bounds check (the index is in
// range by construction) and load the operand of a matmul coalesced.
static bool is_const_i32(const Graph &g, int x, int64_t v) {
  const XNode &n = g.xs[x];
  return n.kind == XK::Const && n.dt == DT::I32 && (int32_t)n.i == (int32_t)v;
}

static bool is_arg0(const Graph &g, int x) { return g.xs[x].kind == XK::Arg && g.xs[x].arg == 0; }

static bool is_div_k_m(const Graph &g, int x, int64_t m) {
  const XNode &n = g.xs[x];
  return n.kind == XK::Bin && n.op == B_DIV && is_arg0(g, n.a) && is_const_i32(g, n.b, m);
}

int transpose_source(const Graph &g, int t) {
  const TNode &n = g.ts[t];
  if (n.kind != TK::Gather || n.shape.size() != 2) return -1;
  const TNode &idx = g.ts[n.a];
  const TNode &src = g.ts[n.b];
  if (src.shape.size() != 2 || idx.kind != TK::Map || g.ts[idx.a].kind != TK::Iota) return -1;
  int64_t m = src.shape[0], nn = src.shape[1];
  if (n.shape[0] != nn || n.shape[1] != m) return -1;
  // add(mul(sub(k, mul(div(k, m), m)), n), div(k, m))
  const XNode &add = g.xs[idx.body];
  if (add.kind != XK::Bin || add.op != B_ADD || !is_div_k_m(g, add.b, m)) return -1;
  const XNode &mul = g.xs[add.a];
  if (mul.kind != XK::Bin || mul.op != B_MUL || !is_const_i32(g, mul.b, nn)) return -1;
  const XNode &sub = g.xs[mul.a];
  if (sub.kind != XK::Bin || sub.op != B_SUB || !is_arg0(g, sub.a)) return -1;
  const XNode &qm = g.xs[sub.b];
  if (qm.kind != XK::Bin || qm.op != B_MUL || !is_div_k_m(g, qm.a, m) || !is_const_i32(g, qm.b, m)) return -1;
  return n.b;
}

Plan fusion_plan(const Graph &g) {
  Plan p;
  p.materialized.assign(g.ts.size(), false);
  std::vector<bool> is_out(g.ts.size(), false);
  for (auto &o : g.outputs) is_out[o.second] = true;
  for (size_t i = 0; i < g.ts.size(); i++) {
    const TNode &t = g.ts[i];
    bool barrier = t.kind == TK::Reduce || t.kind == TK::Scan || t.kind == TK::Scatter || t.kind == TK::Matmul;
    if (t.kind == TK::Param || barrier || is_out[i] || g.fan_out[i] >= 2) {
      p.materialized[i] = true;
      if (t.kind != TK::Param) p.roots.push_back((int)i);
    }
  }
  return p;
}

}  // namespace cchip
