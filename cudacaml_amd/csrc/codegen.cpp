// Graph -> ProgramIR: the fusion inliner, the element-expression printer and
// the gfx950 kernel templates.
//
// The inliner restates Lower's elem/inline_node/expr_of/inputs_of
// (lib/lower/lower.ml:113-197): a materialised node is a load, anything else
// is inlined, so map chains, gathers, transposes and RNG draws fuse into
// whatever consumes them. Each kernel root then picks a CDNA4 template by
// root kind (the role Lower.kernels_of plays at lower.ml:214-958), and the
// host plan keeps the reference's shape (lower.ml:968-1012): allocate params
// then computed buffers, upload, launch root by root, download, free.
//
// The printer keeps the interpreter's arithmetic (cudacaml_backend_interp.ml)
// rather than C's: integer + - * and negation wrap through unsigned, shifts
// mask their count and Shr is logical, Min/Max propagate NaN and order -0
// below +0, float->int casts truncate through int64 then wrap, and an F32
// constant that f32 cannot hold exactly stays a double until an operation
// rounds it (an F32 Const is the unrounded double in the interpreter).

#include <algorithm>
#include <cmath>
#include <cctype>
#include <cstring>
#include <functional>
#include <set>
#include <sstream>
#include <unordered_map>

#include "internal.hpp"

namespace cchip {
namespace {

// ---------------------------------------------------------------------------
// Value classes: how a scalar is carried in the generated code.
// F32D is an f32-typed value that is still a double (an unrounded constant).
// ---------------------------------------------------------------------------

enum class VC { F32, F32D, F64, I32, I64, B };

const char *vc_type(VC c) {
  switch (c) {
    case VC::F32: return "float";
    case VC::F32D: return "double";
    case VC::F64: return "double";
    case VC::I32: return "int";
    case VC::I64: return "long long";
    default: return "bool";
  }
}

VC storage_vc(DT d) {
  switch (d) {
    case DT::F32: return VC::F32;
    case DT::F64: return VC::F64;
    case DT::I32: return VC::I32;
    case DT::I64: return VC::I64;
    default: return VC::B;
  }
}

struct Val {
  std::string s;
  VC c;
};

std::string f32_lit(float v) {
  if (std::isnan(v)) return "__builtin_nanf(\"\")";
  if (std::isinf(v)) return v > 0 ? "__builtin_inff()" : "(-__builtin_inff())";
  char b[64];
  snprintf(b, sizeof b, "%af", (double)v);
  return std::string("(") + b + ")";
}

std::string f64_lit(double v) {
  if (std::isnan(v)) return "__builtin_nan(\"\")";
  if (std::isinf(v)) return v > 0 ? "__builtin_inf()" : "(-__builtin_inf())";
  char b[64];
  snprintf(b, sizeof b, "%a", v);
  return std::string("(") + b + ")";
}

std::string i32_lit(int64_t v) {
  int32_t x = (int32_t)v;
  if (x == INT32_MIN) return "(-2147483647 - 1)";
  return std::to_string(x);
}

std::string i64_lit(int64_t v) {
  if (v == INT64_MIN) return "(-9223372036854775807LL - 1LL)";
  return std::to_string(v) + "LL";
}

// A value in storage form (what a buffer of dtype d holds).
std::string as_storage(const Val &v, DT d) {
  if (d == DT::F32 && v.c == VC::F32D) return "(float)(" + v.s + ")";
  return v.s;
}

std::string as_double(const Val &v) {
  if (v.c == VC::F32) return "(double)(" + v.s + ")";
  return v.s;
}

std::string zero_of(DT d) {
  switch (d) {
    case DT::F32: return "0.0f";
    case DT::F64: return "0.0";
    case DT::I32: return "0";
    case DT::I64: return "0LL";
    default: return "false";
  }
}

// ---------------------------------------------------------------------------
// The element generator: one __device__ function per (root, operand).
// ---------------------------------------------------------------------------

struct ElemFn {
  std::string name;
  std::string code;
  DT dt = DT::F32;
  std::vector<int> ident;  // buffers loaded at the function's own index: passed by value
  std::vector<int> ptrs;   // buffers loaded anywhere else: passed by pointer
  bool uses_err = false;

  // Call with the identity-loaded values given by `identval(buf)`.
  std::string call(const std::string &idx, const std::function<std::string(int)> &identval) const {
    std::string s = name + "(" + idx;
    for (int b : ident) s += ", " + identval(b);
    for (int b : ptrs) s += ", b" + std::to_string(b);
    if (uses_err) s += ", err";
    return s + ")";
  }
  std::string call_scalar(const std::string &idx) const {
    return call(idx, [&](int b) { return "b" + std::to_string(b) + "[" + idx + "]"; });
  }
};

int64_t tune(const char *key, int64_t dflt);

class Gen {
 public:
  Gen(const Graph &g, const Plan &p, const std::vector<int> &buf_of)
      : g_(g), p_(p), buf_of_(buf_of), remat_(tune("remat_broadcast", 1) != 0) {
    for (const XNode &n : g_.xs) {
      int xa = -1, xb = -1;
      if (n.kind == XK::Bin && n.dt == DT::I64 && n.op == B_MUL && zext32(n.a, &xa) && zext32(n.b, &xb)) {
        wide_pairs_.insert({xa, xb});
        wide_pairs_.insert({xb, xa});
      }
    }
  }

  // f(i) = the value of tensor `t` at flat index i. If `inline_root`, t is
  // computed (inlined) even though it is materialised: it is the kernel's
  // own output (lower.ml:120-126).
  // A tensor whose elements all equal one value computed from one-element
  // tensors alone: a broadcast, or a map over such tensors whose body does
  // not use the element index.
  bool uniform(int t) {
    if (uni_.empty()) uni_.assign(g_.ts.size(), -1);
    if (uni_[t] >= 0) return uni_[t] != 0;
    const TNode &n = g_.ts[t];
    bool u = false;
    switch (n.kind) {
      case TK::Broadcast: u = true; break;
      case TK::Reshape: u = uniform(n.a); break;
      case TK::Map: u = uniform(n.a) && !uses_index(n.body); break;
      case TK::Map2: u = uniform(n.a) && uniform(n.b) && !uses_index(n.body); break;
      default: break;
    }
    uni_[t] = u ? 1 : 0;
    return u;
  }
  bool uses_index(int x) const {
    std::vector<int> stack = {x};
    std::vector<char> seen(g_.xs.size(), 0);
    while (!stack.empty()) {
      const int y = stack.back();
      stack.pop_back();
      if (y < 0 || seen[y]) continue;
      seen[y] = 1;
      const XNode &e = g_.xs[y];
      if (e.kind == XK::Index) return true;
      stack.push_back(e.a);
      stack.push_back(e.b);
      stack.push_back(e.c);
    }
    return false;
  }

  ElemFn element_fn(const std::string &name, int t, bool inline_root, bool allow_ident) {
    reset(allow_ident);
    Val idx{"i", VC::I32};
    Val r = inline_root ? inline_node(t, idx) : elem(t, idx);
    ElemFn f;
    f.name = name;
    f.dt = g_.ts[t].dt;
    f.ident = ident_;
    f.ptrs = ptrs_;
    f.uses_err = uses_err_;
    std::ostringstream os;
    os << "__device__ __forceinline__ " << dt_ctype(f.dt) << " " << name << "(const int i";
    for (int b : ident_) os << ", const " << dt_ctype(bufdt(b)) << " a" << b;
    for (int b : ptrs_) os << ", const " << dt_ctype(bufdt(b)) << "* __restrict__ b" << b;
    if (uses_err_) os << ", int* __restrict__ err";
    os << ") {\n" << body_.str() << "  return " << as_storage(r, f.dt) << ";\n}\n";
    f.code = os.str();
    return f;
  }

  // The combine function of a Reduce/Scan: T f(T x0, T x1), Index = 0 as in
  // Lower (lower.ml:278).
  std::string combine_fn(const std::string &name, int body, DT dt) {
    reset(false);
    std::vector<Val> env = {{"x0", storage_vc(dt)}, {"x1", storage_vc(dt)}};
    std::unordered_map<int, Val> memo;
    Val r = expr(body, env, Val{"0", VC::I32}, memo);
    std::ostringstream os;
    os << "__device__ __forceinline__ " << dt_ctype(dt) << " " << name << "(const " << dt_ctype(dt) << " x0, const "
       << dt_ctype(dt) << " x1) {\n"
       << body_.str() << "  return " << as_storage(r, dt) << ";\n}\n";
    return os.str();
  }

  std::string const_fn(const std::string &name, int body, DT dt) {
    reset(false);
    std::unordered_map<int, Val> memo;
    Val r = expr(body, {}, Val{"0", VC::I32}, memo);
    std::ostringstream os;
    os << "__device__ __forceinline__ " << dt_ctype(dt) << " " << name << "() {\n"
       << body_.str() << "  return " << as_storage(r, dt) << ";\n}\n";
    return os.str();
  }

  DT bufdt(int b) const { return bufdt_(b); }
  std::function<DT(int)> bufdt_;

 private:
  const Graph &g_;
  const Plan &p_;
  const std::vector<int> &buf_of_;
  bool remat_;
  std::vector<signed char> uni_;
  std::ostringstream body_;
  int ntmp_ = 0;
  bool allow_ident_ = true;
  std::vector<int> ident_, ptrs_;
  bool uses_err_ = false;
  std::map<std::pair<int, std::string>, Val> tmemo_;
  std::map<std::pair<std::string, std::string>, Val> wide_;  // 64-bit products by operand

  std::set<std::pair<int, int>> wide_pairs_;  // I32 operand pairs of those products

 public:
  // Row scans that also store each row's last element (the row's fold) in
  // a side buffer: scan tensor -> (side buffer, row length); and the
  // gathers that read only those elements (index p * L + L - 1 over the
  // scan's rows), which read the side buffer at p instead. The index
  // strings such a gather passes down map back to their row index and the
  // row length they were made with: another tensor with a side buffer,
  // reached at the same index, reads its buffer only if its rows are as
  // long (through a reshape they need not be).
  std::map<int, std::pair<int, int64_t>> rowlast_;
  std::map<int, int> rowlast_gather_;  // gather tensor -> scan tensor
  // Scatters whose index is a * j + b with a != 0 and every value in range,
  // so that each bin is 0 + its one source value or 0: tensor -> (a, b).
  // A read of such a tensor computes that element from the source at j
  // instead of loading the scatter's buffer.
  std::map<int, std::pair<int64_t, int64_t>> scatter_inline_;

 private:
  std::map<std::string, std::pair<std::string, int64_t>> rowlast_idx_;

  Val wide_product(const Val &a, const Val &b) {
    auto w = wide_.find({a.s, b.s});
    if (w == wide_.end()) w = wide_.find({b.s, a.s});
    if (w != wide_.end()) return w->second;
    Val p = def(VC::I64, "((long long)((cc_u64)(cc_u32)(" + a.s + ") * (cc_u64)(cc_u32)(" + b.s + ")))");
    wide_[{a.s, b.s}] = p;
    return p;
  }

  // x is and(cast I64 (y : I32), 0xFFFFFFFF): *y is the I32 word.
  bool zext32(int x, int *y) const {
    const XNode &n = g_.xs[x];
    if (n.kind != XK::Bin || n.op != B_AND || n.dt != DT::I64) return false;
    const XNode &c = g_.xs[n.b];
    const XNode &e = g_.xs[n.a];
    if (c.kind != XK::Const || c.i != 0xFFFFFFFFLL) return false;
    if (e.kind != XK::Cast || g_.xs[e.a].dt != DT::I32) return false;
    *y = e.a;
    return true;
  }

  void reset(bool allow_ident) {
    body_.str("");
    body_.clear();
    ntmp_ = 0;
    allow_ident_ = allow_ident;
    ident_.clear();
    ptrs_.clear();
    uses_err_ = false;
    tmemo_.clear();
    wide_.clear();
  }

  Val def(VC c, const std::string &rhs) {
    std::string n = "v" + std::to_string(ntmp_++);
    body_ << "  const " << vc_type(c) << " " << n << " = " << rhs << ";\n";
    return {n, c};
  }

  static void add_unique(std::vector<int> &v, int x) {
    for (int y : v)
      if (y == x) return;
    v.push_back(x);
  }

  Val elem(int t, const Val &idx) {
    auto key = std::make_pair(t, idx.s);
    auto it = tmemo_.find(key);
    if (it != tmemo_.end()) return it->second;
    Val r;
    if (p_.materialized[t] && remat_ && uniform(t)) {
      // every element is the same value, computed from one-element tensors:
      // computed here (loop-invariant) in place of reading the tensor's
      // buffer, 4 or 8 bytes an element
      r = inline_node(t, idx);
    } else if (p_.materialized[t] && rowlast_.count(t) && rowlast_idx_.count(idx.s) &&
               rowlast_idx_.at(idx.s).second == rowlast_.at(t).second) {
      // the row's last element, from the scan's side buffer
      const int b = rowlast_.at(t).first;
      add_unique(ptrs_, b);
      r = def(storage_vc(g_.ts[t].dt), "b" + std::to_string(b) + "[" + rowlast_idx_.at(idx.s).first + "]");
    } else if (p_.materialized[t] && scatter_inline_.count(t)) {
      // bin idx of scatter_add(a * j + b, src): 0 + src[j] where idx = a * j
      // + b for some j in range, else 0 (the scatter's own kernel computes
      // the same)
      const TNode &sn = g_.ts[t];
      const std::string A = std::to_string(scatter_inline_.at(t).first);
      const std::string N = std::to_string(g_.ts[sn.a].numel);
      const Val q = def(VC::I32, "(" + idx.s + ") - (" + std::to_string(scatter_inline_.at(t).second) + ")");
      const Val ok = def(VC::B, "(" + q.s + " % (" + A + ")) == 0 && " + q.s + " / (" + A + ") >= 0 && " + q.s +
                                    " / (" + A + ") < " + N);
      const Val j = def(VC::I32, ok.s + " ? " + q.s + " / (" + A + ") : 0");
      const Val v = elem(sn.b, j);
      const std::string z = zero_of(sn.dt);
      r = def(storage_vc(sn.dt), ok.s + " ? (" + z + " + " + as_storage(v, sn.dt) + ") : " + z);
    } else if (p_.materialized[t]) {
      int b = buf_of_[t];
      DT d = g_.ts[t].dt;
      if (allow_ident_ && idx.s == "i") {
        add_unique(ident_, b);
        r = {"a" + std::to_string(b), storage_vc(d)};
      } else {
        add_unique(ptrs_, b);
        r = def(storage_vc(d), "b" + std::to_string(b) + "[" + idx.s + "]");
      }
    } else {
      r = inline_node(t, idx);
    }
    tmemo_[key] = r;
    return r;
  }

  Val inline_node(int t, const Val &idx) {
    const TNode &n = g_.ts[t];
    switch (n.kind) {
      case TK::Iota: return idx;
      case TK::Map: {
        std::unordered_map<int, Val> memo;
        return expr(n.body, {elem(n.a, idx)}, idx, memo);
      }
      case TK::Map2: {
        std::unordered_map<int, Val> memo;
        Val a = elem(n.a, idx);
        Val b = elem(n.b, idx);
        return expr(n.body, {a, b}, idx, memo);
      }
      case TK::Gather: {
        // A gather of the last element of every row of a row scan (index
        // p * L + L - 1, in range by construction) reads the scan's side
        // buffer at p where it reaches the scan's buffer.
        auto rl = rowlast_gather_.find(t);
        if (rl != rowlast_gather_.end()) {
          const int64_t L = rowlast_.at(rl->second).second;
          const std::string jn = "(" + idx.s + " * " + std::to_string(L) + " + " + std::to_string(L - 1) + ")";
          rowlast_idx_[jn] = {idx.s, L};
          return elem(n.b, Val{jn, VC::I32});
        }
        // out[i] = src[idx[i]], bounds-checked against the source extent:
        // the interpreter raises on an index out of range (R8); here the
        // kernel raises a flag the host turns into the same error.
        Val j = elem(n.a, idx);
        const TNode &src = g_.ts[n.b];
        if (transpose_source(g_, t) >= 0 && !p_.materialized[n.a]) return elem(n.b, j);
        uses_err_ = true;
        if (src.numel == 0) {
          body_ << "  cc_flag(err, 1);\n";
          return def(storage_vc(src.dt), zero_of(src.dt));
        }
        std::string jn = "v" + std::to_string(ntmp_++);
        body_ << "  int " << jn << " = " << j.s << ";\n";
        body_ << "  if ((unsigned)" << jn << " >= " << src.numel << "u) { cc_flag(err, 1); " << jn << " = 0; }\n";
        // one element: read at 0 whatever the index (the check above still
        // flags one out of range), so the load and what is computed from it
        // do not depend on the element and leave the kernel's loop (a
        // gradient spreads a whole reduction's adjoint by gather(i / n))
        if (src.numel == 1) return elem(n.b, Val{"0", VC::I32});
        return elem(n.b, Val{jn, VC::I32});
      }
      case TK::Reshape: return elem(n.a, idx);
      case TK::Broadcast: return elem(n.a, Val{"0", VC::I32});
      default:
        throw Failure("Lower: Param/Reduce/Scan/Scatter_add/Matmul must be materialised");
    }
  }

  Val expr(int x, const std::vector<Val> &env, const Val &idx, std::unordered_map<int, Val> &memo) {
    auto it = memo.find(x);
    if (it != memo.end()) return it->second;
    Val r = expr1(x, env, idx, memo);
    memo[x] = r;
    return r;
  }

  Val expr1(int x, const std::vector<Val> &env, const Val &idx, std::unordered_map<int, Val> &memo) {
    const XNode &n = g_.xs[x];
    auto go = [&](int y) { return expr(y, env, idx, memo); };
    switch (n.kind) {
      case XK::Const:
        switch (n.dt) {
          case DT::F32: {
            float f = (float)n.f;
            if ((double)f == n.f || std::isnan(n.f)) return {f32_lit(f), VC::F32};
            return {f64_lit(n.f), VC::F32D};
          }
          case DT::F64: return {f64_lit(n.f), VC::F64};
          case DT::I32: return {i32_lit(n.i), VC::I32};
          case DT::I64: return {i64_lit(n.i), VC::I64};
          default: return {n.i ? "true" : "false", VC::B};
        }
      case XK::Arg:
        if (n.arg >= (int)env.size()) throw Failure(strf("Lower: unbound Arg %d", n.arg));
        return env[n.arg];
      case XK::Index: return idx;
      case XK::Bin: {
        // Rng's mulhilo (rng.ml:20-29): the I64 product of two zero-extended
        // I32 words, and the I32 product of the same words. Both halves come
        // from one 32x32->64 multiply (a single v_mad_u64_u32).
        int xa = -1, xb = -1;
        if (n.dt == DT::I64 && n.op == B_MUL && zext32(n.a, &xa) && zext32(n.b, &xb))
          return wide_product(go(xa), go(xb));
        // A 32-bit XOR of a XOR (Philox's hi ^ ctr ^ key, rng.ml:31-36) is
        // one three-input v_bitop3_b32 (truth table 0x96) on gfx950, where
        // the compiler leaves two v_xor_b32. The inner XOR is only
        // evaluated here if something else uses it. Constant operands are
        // left to the compiler, which folds them.
        if (n.dt == DT::I32 && n.op == B_XOR) {
          for (int side = 0; side < 2; side++) {
            const XNode &in = g_.xs[side ? n.b : n.a];
            int other = side ? n.a : n.b;
            if (in.kind == XK::Bin && in.dt == DT::I32 && in.op == B_XOR && g_.xs[in.a].kind != XK::Const &&
                g_.xs[in.b].kind != XK::Const && g_.xs[other].kind != XK::Const) {
              Val x = go(in.a), y = go(in.b), z = go(other);
              return def(VC::I32, "((int)__builtin_amdgcn_bitop3_b32((cc_u32)(" + x.s + "), (cc_u32)(" + y.s +
                                      "), (cc_u32)(" + z.s + "), 0x96))");
            }
          }
        }
        Val a = go(n.a), b = go(n.b);
        if (n.dt == DT::I32 && n.op == B_MUL && wide_pairs_.count({n.a, n.b})) {
          Val p = wide_product(a, b);
          return def(VC::I32, "((int)(cc_u32)(cc_u64)(" + p.s + "))");
        }
        return binop(n, a, b);
      }
      case XK::Un: return unop(n, go(n.a));
      case XK::Cmp: {
        Val a = go(n.a), b = go(n.b);
        static const char *ops[] = {"==", "!=", "<", "<=", ">", ">="};
        std::string sa = a.s, sb = b.s;
        if (a.c == VC::F32D || b.c == VC::F32D) {
          sa = as_double(a);
          sb = as_double(b);
        }
        return def(VC::B, "(" + sa + " " + ops[n.op] + " " + sb + ")");
      }
      case XK::Logic: {
        Val a = go(n.a), b = go(n.b);
        return def(VC::B, "(" + a.s + (n.op == 0 ? " && " : " || ") + b.s + ")");
      }
      case XK::Not: return def(VC::B, "(!" + go(n.a).s + ")");
      case XK::Select: {
        // Rng.to_unit_interval's unsigned reading of a word (rng.ml:61-67):
        // select (w < 0) ((double)w + 2^32) ((double)w) is exactly
        // (double)(unsigned)w, one v_cvt_f64_u32.
        {
          const XNode &cn = g_.xs[n.a], &tn = g_.xs[n.b], &en = g_.xs[n.c];
          if (n.dt == DT::F64 && cn.kind == XK::Cmp && cn.op == C_LT && g_.xs[cn.a].dt == DT::I32 &&
              g_.xs[cn.b].kind == XK::Const && g_.xs[cn.b].i == 0 && en.kind == XK::Cast && en.dt == DT::F64 &&
              en.a == cn.a && tn.kind == XK::Bin && tn.op == B_ADD && tn.dt == DT::F64 &&
              g_.xs[tn.a].kind == XK::Cast && g_.xs[tn.a].a == cn.a && g_.xs[tn.b].kind == XK::Const &&
              g_.xs[tn.b].f == 4294967296.0)
            return def(VC::F64, "((double)(cc_u32)(" + go(cn.a).s + "))");
        }
        Val c = go(n.a), a = go(n.b), b = go(n.c);
        if (a.c == b.c) return def(a.c, "(" + c.s + " ? " + a.s + " : " + b.s + ")");
        // F32 and F32D meet: keep the exact double.
        return def(VC::F32D, "(" + c.s + " ? " + as_double(a) + " : " + as_double(b) + ")");
      }
      case XK::Cast: return cast(n.dt, g_.xs[n.a].dt, go(n.a));
    }
    throw Failure("codegen: bad expression");
  }

  Val binop(const XNode &n, const Val &a, const Val &b) {
    switch (n.dt) {
      case DT::F32: {
        bool exact = a.c == VC::F32 && b.c == VC::F32;
        static const char *sym[] = {"+", "-", "*", "/"};
        if (n.op <= B_DIV) {
          if (exact) return def(VC::F32, "(" + a.s + " " + sym[n.op] + " " + b.s + ")");
          return def(VC::F32, "(float)(" + as_double(a) + " " + sym[n.op] + " " + as_double(b) + ")");
        }
        const char *fn = n.op == B_MIN ? "cc_min" : "cc_max";
        if (exact) return def(VC::F32, std::string(fn) + "f(" + a.s + ", " + b.s + ")");
        return def(VC::F32, std::string("(float)") + fn + "d(" + as_double(a) + ", " + as_double(b) + ")");
      }
      case DT::F64: {
        static const char *sym[] = {"+", "-", "*", "/"};
        if (n.op <= B_DIV) return def(VC::F64, "(" + a.s + " " + sym[n.op] + " " + b.s + ")");
        return def(VC::F64, std::string(n.op == B_MIN ? "cc_mind(" : "cc_maxd(") + a.s + ", " + b.s + ")");
      }
      case DT::I32:
      case DT::I64: {
        bool w = n.dt == DT::I64;
        const char *T = w ? "long long" : "int";
        const char *U = w ? "cc_u64" : "cc_u32";
        VC vc = w ? VC::I64 : VC::I32;
        auto wrap = [&](const char *sym) {
          return def(vc, std::string("((") + T + ")((" + U + ")(" + a.s + ") " + sym + " (" + U + ")(" + b.s + ")))");
        };
        switch (n.op) {
          case B_ADD: return wrap("+");
          case B_SUB: return wrap("-");
          case B_MUL: return wrap("*");
          case B_DIV: return def(vc, std::string(w ? "cc_divl(" : "cc_divi(") + a.s + ", " + b.s + ")");
          case B_MIN: return def(vc, "((" + a.s + " < " + b.s + ") ? " + a.s + " : " + b.s + ")");
          case B_MAX: return def(vc, "((" + a.s + " > " + b.s + ") ? " + a.s + " : " + b.s + ")");
          case B_AND: return wrap("&");
          case B_OR: return wrap("|");
          case B_XOR: return wrap("^");
          case B_SHL:
          case B_SHR: {
            const char *sym = n.op == B_SHL ? "<<" : ">>";
            const char *mask = w ? "63" : "31";
            return def(vc, std::string("((") + T + ")((" + U + ")(" + a.s + ") " + sym + " ((" + U + ")(" + b.s +
                               ") & " + mask + ")))");
          }
        }
        break;
      }
      default: break;
    }
    throw Failure("codegen: binop on bool");
  }

  Val unop(const XNode &n, const Val &a) {
    static const char *f32n[] = {"", "sqrtf", "cc_expf", "cc_logf", "fabsf", "cc_sinf", "cc_cosf", "cc_erff", "cc_erfinvf"};
    static const char *f64n[] = {"", "sqrt", "exp", "log", "fabs", "sin", "cos", "erf", "cc_erfinv"};
    switch (n.dt) {
      case DT::F32:
        if (n.op == U_NEG) {
          if (a.c == VC::F32) return def(VC::F32, "(-" + a.s + ")");
          return def(VC::F32, "(float)(-" + a.s + ")");
        }
        if (a.c == VC::F32) return def(VC::F32, std::string(f32n[n.op]) + "(" + a.s + ")");
        return def(VC::F32, std::string("(float)") + f64n[n.op] + "(" + a.s + ")");
      case DT::F64:
        if (n.op == U_NEG) return def(VC::F64, "(-" + a.s + ")");
        return def(VC::F64, std::string(f64n[n.op]) + "(" + a.s + ")");
      case DT::I32:
        if (n.op == U_NEG) return def(VC::I32, "((int)(0u - (cc_u32)(" + a.s + ")))");
        return def(VC::I32, "((" + a.s + " < 0) ? (int)(0u - (cc_u32)(" + a.s + ")) : " + a.s + ")");
      case DT::I64:
        if (n.op == U_NEG) return def(VC::I64, "((long long)(0ull - (cc_u64)(" + a.s + ")))");
        return def(VC::I64, "((" + a.s + " < 0) ? (long long)(0ull - (cc_u64)(" + a.s + ")) : " + a.s + ")");
      default: break;
    }
    throw Failure("codegen: unop on bool");
  }

  // R6 (cudacaml_backend_interp.ml:198-237).
  Val cast(DT to, DT from, const Val &a) {
    if (to == from) return a;
    switch (from) {
      case DT::F32:
      case DT::F64: {
        std::string d = as_double(a);
        switch (to) {
          case DT::F32: return def(VC::F32, "(float)(" + d + ")");
          case DT::F64: return def(VC::F64, d);
          case DT::I32: return def(VC::I32, "cc_f2i(" + d + ")");
          case DT::I64: return def(VC::I64, "cc_f2l(" + d + ")");
          default: return def(VC::B, "(" + d + " != 0.0)");
        }
      }
      case DT::I32:
      case DT::I64:
        switch (to) {
          case DT::F32: return def(VC::F32, "(float)(double)(" + a.s + ")");
          case DT::F64: return def(VC::F64, "(double)(" + a.s + ")");
          case DT::I32: return def(VC::I32, "((int)(cc_u32)(cc_u64)(" + a.s + "))");
          case DT::I64: return def(VC::I64, "((long long)(" + a.s + "))");
          default: return def(VC::B, "(" + a.s + " != 0)");
        }
      default:
        switch (to) {
          case DT::F32: return def(VC::F32, "(" + a.s + " ? 1.0f : 0.0f)");
          case DT::F64: return def(VC::F64, "(" + a.s + " ? 1.0 : 0.0)");
          case DT::I32: return def(VC::I32, "(" + a.s + " ? 1 : 0)");
          case DT::I64: return def(VC::I64, "(" + a.s + " ? 1LL : 0LL)");
          default: return a;
        }
    }
  }
};

// ---------------------------------------------------------------------------
// The prelude every generated module starts with.
// ---------------------------------------------------------------------------

const char *kPrelude = R"PRELUDE(// Generated by cchip (Backend_hip) for gfx950.
typedef unsigned int cc_u32;
typedef unsigned long long cc_u64;
template <typename T> struct __attribute__((aligned(4 * sizeof(T)))) cc_v4 { T x, y, z, w; };
// Streaming (non-temporal) 4-wide accesses: they do not displace the lines
// that random-access loads of the same kernel reuse.
template <typename T> __device__ __forceinline__ cc_v4<T> cc_ld4_nt(const T* p) {
  typedef T v4 __attribute__((ext_vector_type(4)));
  const v4 v = __builtin_nontemporal_load((const v4*)p);
  return {v.x, v.y, v.z, v.w};
}
template <typename T> __device__ __forceinline__ void cc_st4_nt(T* p, const cc_v4<T>& r) {
  typedef T v4 __attribute__((ext_vector_type(4)));
  const v4 v = {r.x, r.y, r.z, r.w};
  __builtin_nontemporal_store(v, (v4*)p);
}
template <typename T> struct __attribute__((aligned(2 * sizeof(T)))) cc_v2 { T x, y; };
// Buffer-resource accesses of 16 bytes: a descriptor in scalar registers,
// one shared per-lane byte offset and a uniform offset, so a run of loads
// costs one vector register of addressing; out-of-range loads read zero.
// AUX 2 streams (non-temporal), 0 does not. Word 3 is gfx9's.
typedef unsigned int cc_u32x4 __attribute__((ext_vector_type(4)));
typedef float cc_f4v __attribute__((ext_vector_type(4)));
typedef double cc_d2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t cc_rsrc(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
template <typename T, int AUX> __device__ __forceinline__ cc_v4<T> cc_bld4(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  static_assert(sizeof(T) == 4, "4-byte elements");
  const cc_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, AUX);
  cc_v4<T> o;
  __builtin_memcpy(&o, &v, 16);
  return o;
}
template <typename T, int AUX> __device__ __forceinline__ void cc_bst4(__amdgpu_buffer_rsrc_t r, int voff, int soff, const cc_v4<T>& x) {
  static_assert(sizeof(T) == 4, "4-byte elements");
  cc_u32x4 v;
  __builtin_memcpy(&v, &x, 16);
  __builtin_amdgcn_raw_buffer_store_b128(v, r, voff, soff, AUX);
}
template <typename T> __device__ __forceinline__ cc_v2<T> cc_ld2_nt(const T* p) {
  typedef T v2 __attribute__((ext_vector_type(2)));
  const v2 v = __builtin_nontemporal_load((const v2*)p);
  return {v.x, v.y};
}
template <typename T> __device__ __forceinline__ void cc_st2_nt(T* p, const cc_v2<T>& r) {
  typedef T v2 __attribute__((ext_vector_type(2)));
  const v2 v = {r.x, r.y};
  __builtin_nontemporal_store(v, (v2*)p);
}

// Float.min / Float.max of OCaml: NaN if either operand is NaN, -0 below
// +0. These are IEEE 754-2019 minimum/maximum, which gfx950 executes as
// one v_minimum3_f32 / v_maximum3_f32.
__device__ __forceinline__ float cc_minf(float x, float y) { return __builtin_elementwise_minimum(x, y); }
__device__ __forceinline__ float cc_maxf(float x, float y) { return __builtin_elementwise_maximum(x, y); }
__device__ __forceinline__ double cc_mind(double x, double y) { return __builtin_elementwise_minimum(x, y); }
__device__ __forceinline__ double cc_maxd(double x, double y) { return __builtin_elementwise_maximum(x, y); }
// f32 exp and log as the interpreter computes them: the function in double
// precision, rounded once to float. Both are evaluated in double to within
// a few double ulps, so the rounding to float lands where the interpreter's
// does (checked on every float: no difference from (float)exp((double)x)
// and (float)log((double)x) of the host C library). Each takes about 40
// instructions in a loop (the device library's single-precision calls
// about 20; f64 FMAs issue at the f32 rate here), which the maps over 2^28
// elements that call them hide under their HBM time.
// exp: 2^(h/2) e^r, h = rint(2x / ln 2), r = x - h ln2/2 (ln 2 / 2 in two
// parts; |r| <= 0.174), e^r by its Taylor polynomial to degree 10
// (truncation below 2^-53), times sqrt 2 for odd h. Arguments beyond
// [-150, 130] are clamped: the float result is 0 or +inf there either way.
__device__ __forceinline__ float cc_expf(float x) {
  if (x != x) return x;
  double d = (double)x;
  d = d < -150.0 ? -150.0 : (d > 130.0 ? 130.0 : d);
  const double h = __builtin_rint(d * 2.8853900817779268);
  double r = __builtin_fma(-h, 3.46573590184561908245e-01, d);
  r = __builtin_fma(-h, 9.54107464635293850010e-11, r);
  double p = 1.0 / 3628800.0;
  p = __builtin_fma(p, r, 1.0 / 362880.0);
  p = __builtin_fma(p, r, 1.0 / 40320.0);
  p = __builtin_fma(p, r, 1.0 / 5040.0);
  p = __builtin_fma(p, r, 1.0 / 720.0);
  p = __builtin_fma(p, r, 1.0 / 120.0);
  p = __builtin_fma(p, r, 1.0 / 24.0);
  p = __builtin_fma(p, r, 1.0 / 6.0);
  p = __builtin_fma(p, r, 0.5);
  p = __builtin_fma(p, r, 1.0);
  p = __builtin_fma(p, r, 1.0);
  const int hi = (int)h;
  if (hi & 1) p *= 1.4142135623730951;
  return (float)__builtin_ldexp(p, hi >> 1);
}
// log: x = 2^e m with m in [sqrt(1/2), sqrt(2)) (exact in double, float
// subnormals included), log m = 2 atanh t = 2t + 2t^3 q(t^2) with
// t = (m - 1) / (m + 1), |t| <= 0.172, q to the t^16 term (truncation
// below 2^-50), then e ln 2 + log m.
__device__ __forceinline__ float cc_logf(float x) {
  if (!(x > 0.0f) || x == __builtin_inff()) {
    if (x == 0.0f) return -__builtin_inff();
    return x == __builtin_inff() ? x : __builtin_nanf("");  // +inf; negative or NaN
  }
  const double d = (double)x;
  const cc_u64 b = __builtin_bit_cast(cc_u64, d);
  int e = (int)((b >> 52) & 0x7ff) - 1023;
  double m = __builtin_bit_cast(double, (b & 0x000fffffffffffffull) | 0x3ff0000000000000ull);
  if (m > 1.4142135623730951) {
    m *= 0.5;
    e += 1;
  }
  const double t = (m - 1.0) / (m + 1.0);
  const double t2 = t * t;
  double q = 1.0 / 17.0;
  q = __builtin_fma(q, t2, 1.0 / 15.0);
  q = __builtin_fma(q, t2, 1.0 / 13.0);
  q = __builtin_fma(q, t2, 1.0 / 11.0);
  q = __builtin_fma(q, t2, 1.0 / 9.0);
  q = __builtin_fma(q, t2, 1.0 / 7.0);
  q = __builtin_fma(q, t2, 1.0 / 5.0);
  q = __builtin_fma(q, t2, 1.0 / 3.0);
  const double lm = __builtin_fma(2.0 * t * t2, q, 2.0 * t);
  return (float)__builtin_fma((double)e, 0.6931471805599453, lm);
}
// sin, cos and erf in f32 the same way, through the device library's
// double-precision functions (no benchmark's inner loop calls them).
__device__ __forceinline__ float cc_sinf(float x) { return (float)sin((double)x); }
__device__ __forceinline__ float cc_cosf(float x) { return (float)cos((double)x); }
__device__ __forceinline__ float cc_erff(float x) { return (float)erf((double)x); }
// erfinv in single precision, with the structure of M. Giles,
// "Approximating the erfinv function" (GPU Computing Gems, 2011):
// w = -ln(1 - x^2); erfinv(x) = x p(w - 1) for w < 5, else
// x p'(sqrt(w) - 2.5). The coefficients are this backend's own weighted
// least-squares fits to erfinv(x)/x (degree 9 and 10, relative error below
// 7e-9), evaluated as x c0 + x (u q(u)) so that the leading term is
// rounded once. Against the correctly rounded value it is within 1 ulp on
// every float in (-1, 1) (checked exhaustively on the device). The central
// branch costs 16 instructions: where a wave holds no |x| > 0.9966, the
// tail is skipped.
__device__ __forceinline__ float cc_erfinvf(float x) {
  const float t = __builtin_fmaf(-x, x, 1.0f);
  const float L = __builtin_amdgcn_logf(t);  // log2(1 - x^2), one v_log_f32
  float u, q, c0;
  if (L > -0x1.cda994p+2f) {  // w = -ln2 * L < 5, so |x| < 1: no edge cases here
    u = __builtin_fmaf(L, -0x1.62e43p-1f, -1.0f);
    q = -0x1.333982p-27f;
    q = __builtin_fmaf(q, u, 0x1.352e7cp-23f);
    q = __builtin_fmaf(q, u, -0x1.1f508ap-21f);
    q = __builtin_fmaf(q, u, -0x1.25e432p-18f);
    q = __builtin_fmaf(q, u, 0x1.409c76p-15f);
    q = __builtin_fmaf(q, u, 0x1.a47ad6p-14f);
    q = __builtin_fmaf(q, u, -0x1.377b34p-9f);
    q = __builtin_fmaf(q, u, 0x1.16922p-8f);
    q = __builtin_fmaf(q, u, 0x1.fb8fcep-3f);
    c0 = 0x1.209b9cp+0f;
    // x's sign, also for -0 (the products make +0 there)
    return __builtin_copysignf(__builtin_fmaf(x, c0, x * (u * q)), x);
  } else {
    u = __builtin_sqrtf(L * -0x1.62e43p-1f) - 2.5f;
    q = -0x1.e0580ap-16f;
    q = __builtin_fmaf(q, u, 0x1.3ed67cp-12f);
    q = __builtin_fmaf(q, u, -0x1.5b863ap-10f);
    q = __builtin_fmaf(q, u, 0x1.78d0ep-9f);
    q = __builtin_fmaf(q, u, -0x1.16335ap-9f);
    q = __builtin_fmaf(q, u, -0x1.539096p-8f);
    q = __builtin_fmaf(q, u, 0x1.32b17p-6f);
    q = __builtin_fmaf(q, u, -0x1.fe90dp-6f);
    q = __builtin_fmaf(q, u, 0x1.20466cp-5f);
    q = __builtin_fmaf(q, u, 0x1.f6ec82p-1f);
    c0 = 0x1.2b0042p+1f;
  }
  // the tail also takes |x| >= 1 (log of 0 or of a negative) and NaN
  const float y = __builtin_copysignf(__builtin_fmaf(x, c0, x * (u * q)), x);
  const float ax = __builtin_fabsf(x);
  return ax < 1.0f ? y : (ax == 1.0f ? __builtin_copysignf(__builtin_inff(), x) : __builtin_nanf(""));
}
// erfinv in double precision, with the same structure as cc_erfinvf:
// w = -ln(1 - x^2); erfinv(x) = x p(w - 1) for w < 5, x p1(sqrt(w) - 3)
// for 5 <= w < 16, x p2(sqrt(w) - 5) beyond. The coefficients are this
// backend's own fits to erfinv(x)/x (degrees 17, 17 and 14; relative
// error below 4e-14), and w comes from this function's own logarithm:
// 1 - x^2 = m 2^e with m in [sqrt(1/2), sqrt(2)), ln m = 2 atanh(s) with
// s = (m - 1)/(m + 1) summed to s^19. The coefficients of the logarithm
// and of the central branch (w < 5, nearly every draw) come from a
// constant table, so they load into scalar registers and each Horner step
// is one v_fma_f64; as literals, which no VALU encoding takes at 64 bits,
// every step was a v_mov_b64 and a v_fmac_f64 (f64 MC paths: 3.07 ->
// 3.59 * 10^9 paths/s, same bits). The rare tails keep their literals:
// all of them in the table overflow the scalar registers.
__constant__ double cc_e64k[27] = {
  0x1.af286bca1af28p-5,
  0x1.e1e1e1e1e1e1ep-5,
  0x1.1111111111111p-4,
  0x1.3b13b13b13b14p-4,
  0x1.745d1745d1746p-4,
  0x1.c71c71c71c71cp-4,
  0x1.2492492492492p-3,
  0x1.999999999999ap-3,
  0x1.5555555555555p-2,
  0x1.5fd4a83d5303fp-50,
  -0x1.441d7737d7005p-45,
  0x1.daaa8103bac40p-42,
  -0x1.1c2a201a4a356p-39,
  -0x1.aabd1379244f4p-39,
  0x1.2bac1ac83a37dp-34,
  0x1.f08db44ecf9abp-37,
  -0x1.9f5c30f1ec20fp-29,
  0x1.9f2d0f3cb9727p-28,
  0x1.06aacfd6db79ep-23,
  -0x1.2f73e1e1ad259p-21,
  -0x1.1eedf9e372c45p-18,
  0x1.4075e51ae7966p-15,
  0x1.a3f0f037575bep-14,
  -0x1.3779be7bbdc91p-9,
  0x1.16931130fc047p-8,
  0x1.fb8fccc6063e1p-3,
  0x1.209b9bb73e397p+0};
__device__ __forceinline__ double cc_erfinv(double x) {
  const double t = __builtin_fma(-x, x, 1.0);
  double m = __builtin_amdgcn_frexp_mant(t);
  int e = __builtin_amdgcn_frexp_exp(t);
  if (m < 0x1.6a09e667f3bcdp-1) { m = m + m; e = e - 1; }
  const double f = m - 1.0, d = m + 1.0;
  double r = __builtin_amdgcn_rcp(d);
  r = __builtin_fma(__builtin_fma(-d, r, 1.0), r, r);
  r = __builtin_fma(__builtin_fma(-d, r, 1.0), r, r);
  const double s = f * r, s2 = s * s;
  double a = cc_e64k[0];  // 1/19
  a = __builtin_fma(a, s2, cc_e64k[1]);  // 1/17
  a = __builtin_fma(a, s2, cc_e64k[2]);  // 1/15
  a = __builtin_fma(a, s2, cc_e64k[3]);  // 1/13
  a = __builtin_fma(a, s2, cc_e64k[4]);  // 1/11
  a = __builtin_fma(a, s2, cc_e64k[5]);  // 1/9
  a = __builtin_fma(a, s2, cc_e64k[6]);  // 1/7
  a = __builtin_fma(a, s2, cc_e64k[7]);  // 1/5
  a = __builtin_fma(a, s2, cc_e64k[8]);  // 1/3
  const double lnm = __builtin_fma(s + s, s2 * a, s + s);
  const double de = (double)e;
  const double w = -__builtin_fma(de, 0x1.62e42fefa39efp-1, __builtin_fma(de, 0x1.abc9e3b39803fp-56, lnm));
  double u, q, c0;
  if (t > 0x1.b993fe00d5376p-8) {  // t > e^-5, so w < 5 and |x| < 1: no edge cases here
    u = w - 1.0;
    q = cc_e64k[9];
    q = __builtin_fma(q, u, cc_e64k[10]);
    q = __builtin_fma(q, u, cc_e64k[11]);
    q = __builtin_fma(q, u, cc_e64k[12]);
    q = __builtin_fma(q, u, cc_e64k[13]);
    q = __builtin_fma(q, u, cc_e64k[14]);
    q = __builtin_fma(q, u, cc_e64k[15]);
    q = __builtin_fma(q, u, cc_e64k[16]);
    q = __builtin_fma(q, u, cc_e64k[17]);
    q = __builtin_fma(q, u, cc_e64k[18]);
    q = __builtin_fma(q, u, cc_e64k[19]);
    q = __builtin_fma(q, u, cc_e64k[20]);
    q = __builtin_fma(q, u, cc_e64k[21]);
    q = __builtin_fma(q, u, cc_e64k[22]);
    q = __builtin_fma(q, u, cc_e64k[23]);
    q = __builtin_fma(q, u, cc_e64k[24]);
    q = __builtin_fma(q, u, cc_e64k[25]);
    c0 = cc_e64k[26];
    return __builtin_copysign(__builtin_fma(x, c0, x * (u * q)), x);
  } else if (w < 16.0) {
    u = __builtin_sqrt(w) - 3.0;
    q = -0x1.f6f78b1e45962p-28;
    q = __builtin_fma(q, u, -0x1.65291a0e0614ep-22);
    q = __builtin_fma(q, u, 0x1.b798876d2a805p-20);
    q = __builtin_fma(q, u, -0x1.f088ab5adff9dp-20);
    q = __builtin_fma(q, u, -0x1.72be2022a173dp-18);
    q = __builtin_fma(q, u, 0x1.7055c2fd0ca29p-16);
    q = __builtin_fma(q, u, -0x1.83d25844d1db4p-16);
    q = __builtin_fma(q, u, -0x1.857740e3bbcd1p-15);
    q = __builtin_fma(q, u, 0x1.af29a78ddf842p-13);
    q = __builtin_fma(q, u, -0x1.28e4fa6089a85p-12);
    q = __builtin_fma(q, u, -0x1.384aa31a9136fp-13);
    q = __builtin_fma(q, u, 0x1.84f424156f67ap-10);
    q = __builtin_fma(q, u, -0x1.d2754411716b9p-9);
    q = __builtin_fma(q, u, 0x1.7495875fc62eap-8);
    q = __builtin_fma(q, u, -0x1.f4f1c7334e800p-8);
    q = __builtin_fma(q, u, 0x1.3582c81608189p-7);
    q = __builtin_fma(q, u, 0x1.006dca7a9d03ap+0);
    c0 = 0x1.6a9efbd66ea86p+1;
  } else {
    u = __builtin_sqrt(w) - 5.0;
    q = 0x1.7f9d77becd44dp-30;
    q = __builtin_fma(q, u, -0x1.46c201482688ep-28);
    q = __builtin_fma(q, u, 0x1.0c1ab2bf246fep-27);
    q = __builtin_fma(q, u, -0x1.cfdea2298af79p-27);
    q = __builtin_fma(q, u, 0x1.f1fa914c3ba30p-26);
    q = __builtin_fma(q, u, -0x1.27a66f89781d0p-24);
    q = __builtin_fma(q, u, 0x1.ebf30ad12e6eap-23);
    q = __builtin_fma(q, u, -0x1.0a6d5ab35fc61p-20);
    q = __builtin_fma(q, u, 0x1.2fbcd2fc1a433p-18);
    q = __builtin_fma(q, u, -0x1.4a3504248dcc9p-16);
    q = __builtin_fma(q, u, 0x1.3ebf4f5dc40b3p-14);
    q = __builtin_fma(q, u, -0x1.c2f3694b61557p-13);
    q = __builtin_fma(q, u, -0x1.22ea5df45c621p-13);
    q = __builtin_fma(q, u, 0x1.02a30d1fb9c75p+0);
    c0 = 0x1.3664ddd1ad7fcp+2;
  }
  // the tails also take |x| >= 1 (w is then not finite or garbage) and NaN
  const double y = __builtin_copysign(__builtin_fma(x, c0, x * (u * q)), x);
  const double ax = __builtin_fabs(x);
  return ax < 1.0 ? y : (ax == 1.0 ? __builtin_copysign(__builtin_inf(), x) : __builtin_nan(""));
}
// Int32.div / Int64.div: truncation, min_int / -1 wraps. Division by zero
// raises in the interpreter; on the device it yields 0.
__device__ __forceinline__ int cc_divi(int a, int b) {
  return b == 0 ? 0 : (b == -1 ? (int)(0u - (cc_u32)a) : a / b);
}
__device__ __forceinline__ long long cc_divl(long long a, long long b) {
  return b == 0 ? 0 : (b == -1 ? (long long)(0ull - (cc_u64)a) : a / b);
}
// Int64.of_float (truncation; NaN and out-of-range give min_int as the
// x86-64 conversion does), then Int64.to_int32 (wrap).
__device__ __forceinline__ long long cc_f2l(double x) {
  return (x != x || x >= 9223372036854775808.0 || x < -9223372036854775808.0) ? (long long)0x8000000000000000ull
                                                                              : (long long)x;
}
__device__ __forceinline__ int cc_f2i(double x) { return (int)(cc_u32)(cc_u64)cc_f2l(x); }
__device__ __forceinline__ void cc_flag(int* err, int code) {
  __hip_atomic_fetch_or(err, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void cc_atomic_add(float* p, float v) { unsafeAtomicAdd(p, v); }
__device__ __forceinline__ void cc_atomic_add(double* p, double v) { unsafeAtomicAdd(p, v); }
__device__ __forceinline__ void cc_atomic_add(int* p, int v) { atomicAdd(p, v); }
// LDS accumulation. The native float LDS atomic add runs about four times
// slower than a compare-and-swap loop on gfx950, so floats use the loop;
// every round at least one contending lane succeeds, so it terminates.
__device__ __forceinline__ void cc_lds_add(int* p, int v) {
  __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void cc_lds_add(float* p, float v) {
  unsigned* const q = (unsigned*)p;
  unsigned seen = *q;
  while (true) {
    unsigned cur = seen;
    if (__hip_atomic_compare_exchange_strong(q, &cur, __float_as_uint(__uint_as_float(seen) + v), __ATOMIC_RELAXED,
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) break;
    seen = cur;
  }
}
__device__ __forceinline__ void cc_lds_add(double* p, double v) {
  unsigned long long* const q = (unsigned long long*)p;
  unsigned long long seen = *q;
  while (true) {
    unsigned long long cur = seen;
    if (__hip_atomic_compare_exchange_strong(q, &cur,
                                             (unsigned long long)__double_as_longlong(__longlong_as_double((long long)seen) + v),
                                             __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) break;
    seen = cur;
  }
}
// Exclusive prefix of v over a workgroup of NW wave64s; *total gets the
// sum. ws: NW ints of LDS. Every thread of the workgroup must call it.
template <int NW>
__device__ __forceinline__ int cc_wg_exscan_n(int v, int* ws, int* total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(incl, off);
    if (lane >= off) incl += o;
  }
  if (lane == 63) ws[wv] = incl;
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NW; w++) {
    const int t = ws[w];
    if (w < wv) base += t;
    tot += t;
  }
  *total = tot;
  __syncthreads();
  return base + incl - v;
}
// The same over a 256-thread workgroup.
__device__ __forceinline__ int cc_wg_exscan(int v, int* ws, int* total) { return cc_wg_exscan_n<4>(v, ws, total); }
__device__ __forceinline__ cc_u64 cc_bits(float v) { return (cc_u64)__float_as_uint(v); }
__device__ __forceinline__ cc_u64 cc_bits(int v) { return (cc_u64)(cc_u32)v; }
__device__ __forceinline__ cc_u64 cc_bits(double v) { return (cc_u64)__double_as_longlong(v); }
__device__ __forceinline__ cc_u64 cc_bits(long long v) { return (cc_u64)v; }
template <typename T> __device__ __forceinline__ T cc_from_bits(cc_u64 b);
template <> __device__ __forceinline__ float cc_from_bits<float>(cc_u64 b) { return __uint_as_float((cc_u32)b); }
template <> __device__ __forceinline__ int cc_from_bits<int>(cc_u64 b) { return (int)(cc_u32)b; }
template <> __device__ __forceinline__ double cc_from_bits<double>(cc_u64 b) { return __longlong_as_double((long long)b); }
template <> __device__ __forceinline__ long long cc_from_bits<long long>(cc_u64 b) { return (long long)b; }
)PRELUDE";

std::string subst(std::string s, const std::map<std::string, std::string> &vars) {
  for (auto &kv : vars) {
    std::string key = "${" + kv.first + "}";
    size_t pos = 0;
    while ((pos = s.find(key, pos)) != std::string::npos) {
      s.replace(pos, key.size(), kv.second);
      pos += kv.second.size();
    }
  }
  return s;
}

int64_t pow2ceil(int64_t n) {
  int64_t p = 1;
  while (p < n) p <<= 1;
  return p;
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Launch-shape knobs for sweeps: CCHIP_TUNE="key=value,key=value". Every
// key has a default that is the shipped configuration; a knob only changes
// tile sizes and grid shapes, never what is computed, except that the
// grouping knobs of float reductions (rr_tree, fuse_reduce) change their
// last bits within the reduction tolerance.
int64_t tune(const char *key, int64_t dflt) {
  const char *env = getenv("CCHIP_TUNE");
  if (!env) return dflt;
  std::string s = env, k = std::string(key) + "=";
  size_t p = 0;
  while (p < s.size()) {
    size_t e = s.find(',', p);
    if (e == std::string::npos) e = s.size();
    std::string item = s.substr(p, e - p);
    if (item.compare(0, k.size(), k) == 0) return strtoll(item.c_str() + k.size(), nullptr, 10);
    p = e + 1;
  }
  return dflt;
}

// Whether generated code calls one of the f32 functions computed in double.
bool calls_f32_fn(const std::string &code) {
  for (const char *fn : {"cc_expf(", "cc_logf(", "cc_sinf(", "cc_cosf(", "cc_erff(", "cc_erfinvf("})
    if (code.find(fn) != std::string::npos) return true;
  return false;
}

// Whether generated code loads a buffer (b<k>[...]) at anything but index 0.
bool varying_load(const std::string &code) {
  for (size_t q = code.find('b'); q != std::string::npos; q = code.find('b', q + 1)) {
    if (q > 0 && (std::isalnum((unsigned char)code[q - 1]) || code[q - 1] == '_')) continue;
    size_t e = q + 1;
    while (e < code.size() && std::isdigit((unsigned char)code[e])) e++;
    if (e == q + 1 || e >= code.size() || code[e] != '[') continue;
    if (code.compare(e, 3, "[0]") != 0) return true;
  }
  return false;
}

// Accumulation with an empty flag (`acc`, `has` in scope): x is folded in on
// the right; the first value is taken as is.
std::string fold_in(const std::string &cmb, const std::string &T, const std::string &x) {
  return "{ const " + T + " x_ = " + x + "; acc = has ? " + cmb + "(acc, x_) : x_; has = true; }";
}

// As fold_in, but only where `cond` holds, without a branch: the value is
// folded and then selected, so the loads that feed it cannot be sunk into a
// conditional block (which would serialise them behind one another).
std::string fold_in_if(const std::string &cmb, const std::string &T, const std::string &x, const std::string &cond) {
  return "{ const " + T + " x_ = " + x + "; const bool ok_ = " + cond + "; const " + T + " y_ = has ? " + cmb +
         "(acc, x_) : x_; acc = ok_ ? y_ : acc; has = has || ok_; }";
}

// One butterfly step over (acc, has): the lower lane's value stays on the left.
std::string xor_combine(const std::string &cmb, const std::string &T, const std::string &off) {
  return "{ const " + T + " o_ = __shfl_xor(acc, " + off + "); const bool oh_ = __shfl_xor((int)has, " + off +
         ") != 0; if (oh_) { acc = has ? " + cmb + "(acc, o_) : o_; has = true; } }";
}

// Look-back fold over lanes (`w`, `hw` in scope; lane 0 is the nearest
// tile): lanes further away are earlier in the row, so they go on the left.
std::string lookback_tree(const std::string &cmb, const std::string &T) {
  std::string r;
  for (int off = 1; off < 64; off *= 2)
    r += "        { const " + T + " o = __shfl_down(w, " + std::to_string(off) + "); const bool oh = __shfl_down((int)hw, " +
         std::to_string(off) + ") != 0;\n          if ((lane & " + std::to_string(2 * off - 1) +
         ") == 0 && oh) { w = hw ? " + cmb + "(o, w) : o; hw = true; } }\n";
  return r;
}

// The look-back's fallback: the aggregate `agg` of tile `q`, folded by the
// calling wave: lane l folds its contiguous share of the tile left to
// right, then the lanes' partials are combined with lower lanes on the
// left (a row's first tile starts from init, as the tile itself does).
// Few registers are live, so the fallback does not cost the main path its
// occupancy; it is only taken when a predecessor never publishes.
// Declares tq (q's index within its row).
std::string tile_fold(const ElemFn &f, const std::string &cmb, const std::string &ini, const std::string &T, int64_t U,
                      int64_t tpr, int64_t len, int64_t tile) {
  (void)U;
  const int64_t C = cdiv(tile, 64);
  std::ostringstream a;
  a << "            const int rq = q / " << tpr << ", tq = q - rq * " << tpr << ";\n"
    << "            const int bq = rq * " << len << " + tq * " << tile << ";\n"
    << "            const int lq = min(" << tile << ", " << len << " - tq * " << tile << ");\n"
    << "            " << T << " w = " << ini << "();\n"
    << "            bool hw = false;\n"
    << "            for (int e = lane * " << C << "; e < min(lq, (lane + 1) * " << C << "); e++) {\n"
    << "              const " << T << " x = " << f.call_scalar("(bq + e)") << ";\n"
    << "              w = hw ? " << cmb << "(w, x) : x;\n"
    << "              hw = true;\n"
    << "            }\n";
  for (int off = 1; off < 64; off *= 2)
    a << "            { const " << T << " o = __shfl_down(w, " << off << "); const bool oh = __shfl_down((int)hw, " << off
      << ") != 0;\n"
      << "              if ((lane & " << 2 * off - 1 << ") == 0 && oh) { w = hw ? " << cmb
      << "(w, o) : o; hw = true; } }\n";
  a << "            " << T << " agg = __shfl(w, 0);\n"
    << "            if (tq == 0) agg = " << cmb << "(" << ini << "(), agg);\n";
  return a.str();
}

// ---------------------------------------------------------------------------
// The lowering proper
// ---------------------------------------------------------------------------

struct Lowering {
  const Graph &g;
  Plan plan;
  ProgramIR prog;
  std::vector<int> buf_of;  // tensor position -> buffer index (-1 if none)
  std::ostringstream src;
  Gen gen;
  bool need_err = false;

  // One partition pass of the LDS scatter: per-chunk bucket offsets
  // (`cnt`), bucket starts (`start`), the pairs grouped by bucket (`key`,
  // `val`), and, kept for a gather back, each element's slot within its
  // tile (`slot`) and per tile its runs' starts (`meta`).
  struct PassOut {
    int cnt = -1, start = -1, key = -1, val = -1, slot = -1, meta = -1, nbuf = -1;
    int64_t G = 0, C = 0, TILE = 0, TPC = 0, PB = 0;
    std::string nvalid;
    bool first = false;
    // Tile-local layout: each tile's pairs stay in the tile's own region of
    // RS elements, grouped by bucket, every bucket's run starting at a
    // multiple of 8; `meta` holds per bucket and tile {run start within the
    // region, count} ([PB + 1][NTT] int2, row PB: {the region's used
    // length, 0}). No count or offset passes.
    bool local = false;
    int64_t RS = 0, NTT = 0;
    // Windows (the slice pass of two levels, tile-local): a tile is a
    // window of TILE elements of one super-slice's run in the coarse output
    // (`wstart`: the coarse pass's super-slice starts, P1 of them), so its
    // buckets are that super-slice's 64 slices; NTT bounds the windows.
    bool windows = false;
    int wstart = -1, wtab = -1;  // wtab: each super-slice's first window, and the total
    int64_t P1 = 0;
    // per tile: K, the K + 1 tile-local starts of its non-empty buckets
    // (the last is the tile's total), their K run starts in the pair arrays
    int64_t kmax() const { return std::min(TILE, PB); }
    int64_t meta_stride() const { return 2 * kmax() + 2; }
  };
  // A scatter_add whose partition a later gather(idx, h) root reads back
  // through: scatter tensor -> gather root (found before lowering), and the
  // scatter's passes once it has been lowered that way.
  struct GatherBack {
    PassOut fin, coarse;
    int64_t S = 0, P = 0, B = 0, N = 0;
    int h = -1;
    bool fused = false;  // the accumulate already put h[key] in the pairs
  };
  std::map<int, int> gbp_root_of;
  std::map<int, GatherBack> gather_back;
  // scratch buffers freed after a later root than the one that made them
  std::map<int, int> free_after;
  // Whole-tensor reductions of the previous root's map output, folded inside
  // that map's kernel: map root -> reduce root, and reduce root -> the
  // partials (one value a map wave), their has-element flags and count.
  struct FusedPartials {
    int part = -1, flags = -1;
    int64_t count = 0;
  };
  std::map<int, int> fused_red_of_map;
  std::map<int, FusedPartials> fused_part_of_red;
  // bytes a map kernel reads for its folded reduction's expression beyond
  // its own loads
  std::map<int, int64_t> map_extra_moved;
  // Map roots whose output nothing reads once their reduction folds in
  // their kernel (set by lower_program for a second lowering): their
  // kernels store nothing but the partials, and their buffers are elided.
  std::set<int> no_store;
  // Row roots over one tensor fused into one kernel: a row scan that takes
  // the one-workgroup-a-row tile template, and the reductions of the same
  // tensor's rows that fold as a tree. The group's first root in the plan
  // (lead) launches the kernel; the others launch nothing.
  std::map<int, std::vector<int>> sib_reds;  // scan root -> its reductions
  std::map<int, int> sib_lead;               // first root of a group -> scan root
  std::set<int> sib_member;                  // every root of a group but the lead
  // A reduction that folds the same rows with the same combine and init as
  // a scan is the scan's last element of every row: the scan stores those
  // into the reduction's buffer (its row-last side buffer) and the
  // reduction launches nothing. It is part of the scan's group.
  std::map<int, int> same_fold_of;  // scan root -> reduce root
  std::set<int> same_fold_red;

  explicit Lowering(const Graph &gr) : g(gr), plan(fusion_plan(gr)), gen(gr, plan, buf_of) {
    gen.bufdt_ = [this](int b) { return prog.bufs[b].dt; };
  }

  int add_buf(const std::string &name, DT dt, int64_t numel, BufRole role) {
    BufSpec b;
    b.name = name;
    b.dt = dt;
    b.numel = numel;
    b.role = role;
    prog.bufs.push_back(b);
    return (int)prog.bufs.size() - 1;
  }

  int err_buf() {
    if (prog.err_buf < 0) prog.err_buf = add_buf("err", DT::I32, 1, BufRole::Err);
    return prog.err_buf;
  }

  std::string ty(int b) const { return dt_ctype(prog.bufs[b].dt); }

  // Kernel parameter list: every buffer the element functions read, then
  // the written buffers, then the error word.
  struct Params {
    std::vector<int> in, out;
    bool err = false;
  };

  static void add_in(Params &p, const ElemFn &f) {
    auto add = [&](int b) {
      for (int x : p.in)
        if (x == b) return;
      p.in.push_back(b);
    };
    for (int b : f.ident) add(b);
    for (int b : f.ptrs) add(b);
    if (f.uses_err) p.err = true;
  }

  std::string param_list(const Params &p, std::vector<int> &args) {
    std::ostringstream os;
    bool first = true;
    auto sep = [&]() {
      if (!first) os << ", ";
      first = false;
    };
    for (int b : p.in) {
      sep();
      os << "const " << ty(b) << "* __restrict__ b" << b;
      args.push_back(b);
    }
    for (int b : p.out) {
      sep();
      os << ty(b) << "* __restrict__ b" << b;
      args.push_back(b);
    }
    if (p.err) {
      sep();
      os << "int* __restrict__ err";
      args.push_back(err_buf());
      need_err = true;
    }
    return os.str();
  }

  int add_kernel(const std::string &name, const std::vector<int> &args, int grid, int block, const std::string &role,
                 int grid_y = 1) {
    KernelSpec k;
    k.name = name;
    k.args = args;
    k.grid = std::max(1, grid);
    k.grid_y = std::max(1, grid_y);
    k.block = block;
    k.role = role;
    prog.kernels.push_back(k);
    return (int)prog.kernels.size() - 1;
  }

  // Loads of the identity-indexed buffers of `f` as 4-wide vectors at `i`.
  // One vector load per identity-indexed input: `w` elements (4, or 2 for
  // the 16-byte groups of 8-byte types) at index i.
  static std::string vec_loads(const ElemFn &f, const std::string &i, const std::string &indent,
                               const std::function<std::string(int)> &tyof, bool nt = false, int w = 4) {
    std::string s, V = "cc_v" + std::to_string(w), ld = "cc_ld" + std::to_string(w) + "_nt(";
    for (int b : f.ident) {
      std::string bb = "b" + std::to_string(b);
      if (nt)
        s += indent + "const " + V + "<" + tyof(b) + "> l" + std::to_string(b) + " = " + ld + bb + " + " + i + ");\n";
      else
        s += indent + "const " + V + "<" + tyof(b) + "> l" + std::to_string(b) + " = *(const " + V + "<" + tyof(b) +
             ">*)(" + bb + " + " + i + ");\n";
    }
    return s;
  }

  static std::string lane_call(const ElemFn &f, const std::string &i, int k) {
    static const char *comp[] = {"x", "y", "z", "w"};
    std::string idx = k == 0 ? i : "(" + i + " + " + std::to_string(k) + ")";
    return f.call(idx, [&](int b) { return "l" + std::to_string(b) + "." + comp[k]; });
  }

  std::function<std::string(int)> tyof() {
    return [this](int b) { return ty(b); };
  }

  // ---- Algorithmic bytes per root ------------------------------------------
  // Bytes an element function reads when evaluated at n indices: a buffer
  // read at the element's own index contributes the elements read; one read
  // anywhere else (a gather) one element per evaluation, at most the
  // buffer; a one-element buffer (a scalar or a broadcast source) one.
  // Only buffers the function's result (or a side effect such as a bounds
  // flag) depends on count: loads of sub-expressions that end up unused are
  // dropped by the compiler, so they move no bytes.
  int64_t fn_bytes(const ElemFn &f, int64_t n) const {
    std::set<int> ident, ptrs;
    live_buffers(f.code, ident, ptrs);
    int64_t b = 0;
    for (int x : f.ident)
      if (ident.count(x)) b += std::min(prog.bufs[x].numel, n) * dt_size(prog.bufs[x].dt);
    for (int x : f.ptrs) {
      if (!ptrs.count(x) || ident.count(x)) continue;
      int64_t e = prog.bufs[x].numel <= 1 ? prog.bufs[x].numel : std::min(prog.bufs[x].numel, n);
      b += e * dt_size(prog.bufs[x].dt);
    }
    return b;
  }

  // Kernels that move more than the 256 MB MALL cannot keep their working
  // set in it: they stream (non-temporal loads and stores), which keeps
  // their lines from evicting other data and saves the write-back of dirty
  // lines a later kernel would otherwise pay. Below the MALL's size plain
  // accesses win (the data is reused from it).
  static bool streams(int64_t bytes) { return bytes > tune("nt_bytes", int64_t(256) << 20); }
  // The row, look-back and reduction templates give each lane groups of 4
  // consecutive elements; for 8-byte types one group is two interleaved
  // 16-byte accesses, which stream badly (measured: a 2 GiB f64 fill at
  // 2.2 TB/s streaming against 6.3 TB/s plain). Those templates stream
  // 4-byte operands only.
  bool narrow(const ElemFn &f, DT out) const {
    if (dt_size(out) > 4) return false;
    for (int b : f.ident)
      if (dt_size(prog.bufs[b].dt) > 4) return false;
    return true;
  }

  // Liveness over an element function's body: each line either defines a
  // temporary vN or is a statement kept for its effect; the return value
  // and those statements are the roots. Collects the aN (value parameters)
  // and bN (buffer pointers) the live lines use.
  static void live_buffers(const std::string &code, std::set<int> &ident, std::set<int> &ptrs) {
    auto tokens = [](const std::string &line) {
      std::vector<std::string> out;
      size_t i = 0;
      while (i < line.size()) {
        char c = line[i];
        if (isdigit((unsigned char)c)) {  // numeric literal, hex floats included
          while (i < line.size() && (isalnum((unsigned char)line[i]) || line[i] == '.' || line[i] == '_')) i++;
        } else if (isalpha((unsigned char)c) || c == '_') {
          size_t j = i;
          while (j < line.size() && (isalnum((unsigned char)line[j]) || line[j] == '_')) j++;
          out.push_back(line.substr(i, j - i));
          i = j;
        } else {
          i++;
        }
      }
      return out;
    };
    auto kind = [](const std::string &t, char k) {
      if (t.size() < 2 || t[0] != k) return false;
      for (size_t i = 1; i < t.size(); i++)
        if (!isdigit((unsigned char)t[i])) return false;
      return true;
    };
    size_t body = code.find(") {\n");
    if (body == std::string::npos) return;
    std::map<std::string, std::vector<std::string>> defs;
    std::vector<std::string> work;
    size_t pos = body + 4;
    while (pos < code.size()) {
      size_t e = code.find('\n', pos);
      if (e == std::string::npos) e = code.size();
      std::string line = code.substr(pos, e - pos);
      pos = e + 1;
      std::vector<std::string> t = tokens(line);
      if (t.empty()) continue;
      // "const T vN = ..." or "T vN = ...": a definition
      size_t eq = line.find(" = ");
      std::string def;
      if (eq != std::string::npos && line.find("if ") == std::string::npos) {
        std::vector<std::string> lhs = tokens(line.substr(0, eq));
        if (!lhs.empty() && kind(lhs.back(), 'v')) def = lhs.back();
      }
      if (!def.empty()) {
        std::vector<std::string> rhs = tokens(line.substr(eq + 3));
        defs[def].insert(defs[def].end(), rhs.begin(), rhs.end());
      } else {
        for (auto &x : t) work.push_back(x);  // return statement or effect
      }
    }
    std::set<std::string> seen;
    while (!work.empty()) {
      std::string x = work.back();
      work.pop_back();
      if (!seen.insert(x).second) continue;
      if (kind(x, 'a')) ident.insert(atoi(x.c_str() + 1));
      if (kind(x, 'b')) ptrs.insert(atoi(x.c_str() + 1));
      auto it = defs.find(x);
      if (it != defs.end())
        for (auto &y : it->second) work.push_back(y);
    }
  }

  // A fused group of sibling row roots: the kernel carries every member
  // root's algorithmic bytes, and moves the shared tensor's reads once plus
  // every member's output.
  void attribute_group_bytes(int scan, const std::vector<int> &reds, const std::vector<int> &ks) {
    if (ks.empty()) return;
    const TNode &sn = g.ts[scan];
    int64_t algo = root_bytes(scan), moved = fn_bytes(gen.element_fn("ab_", sn.a, false, true), g.ts[sn.a].numel) +
                                              sn.numel * dt_size(sn.dt);
    std::vector<int> all = reds;
    const auto sf = same_fold_of.find(scan);
    if (sf != same_fold_of.end()) all.push_back(sf->second);
    for (int r : all) {
      algo += root_bytes(r);
      moved += g.ts[r].numel * dt_size(g.ts[r].dt);
    }
    prog.kernels[ks.back()].algo_bytes = algo;
    prog.kernels[ks.back()].moved_bytes = moved;
  }

  void attribute_bytes(int r, const std::vector<int> &ks) {
    if (ks.empty()) return;
    const TNode &n = g.ts[r];
    const int64_t out = n.numel * dt_size(n.dt);
    const int64_t bytes = root_bytes(r);
    static const char *helpers[] = {"scan_init",          "scatter_zero",   "scatter_count",  "scatter_colscan",
                                    "scatter_bscan",      "scatter_accumulate", "scatter_reduce", "matmul_ksum",
                                    "reduce_split_fold",  "scatter_coarse",     "gather_slices",  "scatter_windows"};
    int main = ks.back();
    for (int k : ks) {
      bool helper = false;
      for (const char *h : helpers) helper |= prog.kernels[k].role == h;
      if (!helper) main = k;
    }
    prog.kernels[main].algo_bytes = bytes;
    // a reduction folded inside its input's map reads only the partials
    // (scratch): it moves its output alone; a scan with a side buffer of
    // row-last elements also writes that
    prog.kernels[main].moved_bytes = n.kind == TK::Reduce && fused_part_of_red.count(r) ? out : bytes;
    const auto em = map_extra_moved.find(r);
    if (em != map_extra_moved.end()) prog.kernels[main].moved_bytes += em->second;
    if (no_store.count(r)) prog.kernels[main].moved_bytes -= out;
    const auto rl = gen.rowlast_.find(r);
    if (rl != gen.rowlast_.end())
      prog.kernels[main].moved_bytes += prog.bufs[rl->second.first].bytes();
  }

  // The fusion plan's algorithmic bytes of root r: each element it reads
  // counted once, its output written once.
  int64_t root_bytes(int r) {
    const TNode &n = g.ts[r];
    const int64_t out = n.numel * dt_size(n.dt);
    int64_t bytes = 0;
    switch (n.kind) {
      case TK::Reduce:
      case TK::Scan: bytes = fn_bytes(gen.element_fn("ab_", n.a, false, true), g.ts[n.a].numel) + out; break;
      case TK::Scatter: {
        int64_t N = g.ts[n.a].numel;
        bytes = fn_bytes(gen.element_fn("ab_", n.a, false, true), N) +
                fn_bytes(gen.element_fn("ab_", n.b, false, true), N) + out;
        break;
      }
      case TK::Matmul: {
        int64_t M = n.shape[0], N = n.shape[1], K = g.ts[n.a].shape[1];
        bytes = fn_bytes(gen.element_fn("ab_", n.a, false, true), M * K) +
                fn_bytes(gen.element_fn("ab_", n.b, false, true), K * N) + out;
        break;
      }
      default: bytes = fn_bytes(gen.element_fn("ab_", r, true, true), n.numel) + out;
    }
    return bytes;
  }

  // ---- element-wise root (K1 -> vectorised map, one 16-byte group a lane) ---
  std::vector<int> lower_map(int t) {
    const TNode &n = g.ts[t];
    std::string kname = "k_" + std::to_string(n.id);
    int out = buf_of[t];
    ElemFn f = gen.element_fn("f_" + std::to_string(n.id), t, true, true);
    src << f.code;
    // A whole-tensor reduction folded here (below). When its input is an
    // element-wise expression of this output and of other tensors at the
    // same index rather than the output itself: that expression's element
    // function (fe), and fx, the same function with only the tensors it
    // loads beyond this map's own loads and output.
    const auto fr = fused_red_of_map.find(t);
    const bool fuse = fr != fused_red_of_map.end();
    const bool fexpr = fuse && g.ts[fr->second].a != t;
    ElemFn fe, fx;
    if (fexpr) {
      fe = gen.element_fn("fe_" + std::to_string(g.ts[fr->second].id), g.ts[fr->second].a, false, true);
      src << fe.code;
      fx = fe;
      fx.ident.clear();
      for (int b : fe.ident)
        if (b != out && std::find(f.ident.begin(), f.ident.end(), b) == f.ident.end()) fx.ident.push_back(b);
    }
    // a side buffer of each row's last element (Gen::rowlast_), if a later
    // gather reads only those
    const auto sd = gen.rowlast_.find(t);
    const int side = sd != gen.rowlast_.end() ? sd->second.first : -1;
    const int64_t SL_ = side >= 0 ? sd->second.second : 0;
    const bool store = !no_store.count(t);
    if (!store) prog.bufs[out].elided = true;
    Params p;
    add_in(p, f);
    if (fexpr) add_in(p, fx);
    if (store) p.out.push_back(out);
    if (side >= 0) p.out.push_back(side);
    std::vector<int> args;
    std::string params = param_list(p, args);
    int64_t N = n.numel;
    if (N == 0) return {};
    // the side store of element e holding v
    auto side_st = [&](const std::string &e, const std::string &v) {
      return "if ((" + e + ") % " + std::to_string(SL_) + " == " + std::to_string(SL_ - 1) + ") b" +
             std::to_string(side) + "[(" + e + ") / " + std::to_string(SL_) + "] = " + v + ";";
    };
    std::string T = dt_ctype(n.dt);
    // Non-temporal streaming accesses when the kernel also gathers or moves
    // more than the MALL holds (mode 1), always (2) or never (0).
    int64_t nt_mode = tune("map_nt", 1);
    bool nt = nt_mode == 2 || (nt_mode == 1 && (!f.ptrs.empty() || !fx.ptrs.empty() ||
                                                 streams(fn_bytes(f, N) + (fexpr ? fn_bytes(fx, N) : 0) +
                                                         N * dt_size(n.dt))));
    if (n.dt == DT::BOOL) nt = false;
    for (int b : f.ident) nt = nt && prog.bufs[b].dt != DT::BOOL;
    for (int b : fx.ident) nt = nt && prog.bufs[b].dt != DT::BOOL;
    // Loads and stores separately: -1 follows map_nt, 0 plain, 1 streaming.
    // A map that reads no stream (a fill from scalars) stores plainly: that
    // measured faster for write-only kernels (1 GiB: 168 us against 190).
    int64_t ntl_k = tune("map_ntl", -1), nts_k = tune("map_nts", -1);
    bool ntl = ntl_k < 0 ? nt : ntl_k != 0;
    bool nts = nts_k < 0 ? nt && (nt_mode == 2 || !f.ident.empty()) : nts_k != 0;
    if (n.dt == DT::BOOL) nts = false;
    for (int b : f.ident) ntl = ntl && prog.bufs[b].dt != DT::BOOL;
    for (int b : fx.ident) ntl = ntl && prog.bufs[b].dt != DT::BOOL;
    // Elements per thread and access: 16 bytes of the widest type, so each
    // wave instruction covers one contiguous run (4 for 4-byte types, 2 when
    // any operand is 8 bytes wide).
    int G = dt_size(n.dt) == 8 ? 2 : 4;
    for (int b : f.ident)
      if (dt_size(prog.bufs[b].dt) == 8) G = 2;
    for (int b : fx.ident)
      if (dt_size(prog.bufs[b].dt) == 8) G = 2;
    const std::string VG = "cc_v" + std::to_string(G);
    // Groups per lane per iteration. An element function with a long
    // dependent chain (a Horner recurrence) needs about four independent
    // chains per lane to keep the VALU busy: a group of 4-byte elements
    // has four, a group of 8-byte ones two, so heavy functions over 8-byte
    // groups take two groups, which the scheduler interleaves (degree-64
    // Horner in f64: 80 -> 75 us per 2^24; in f32 a second group measured
    // slower, 105 -> 108 us).
    // The extra group's index is clamped to the last group, and its store
    // is unconditional too: a lane past the end recomputes the last group
    // and stores the same values its owner stores. A guarded store would
    // let the compiler sink the whole second chain under the guard.
    //
    // A lighter function that calls one of the f32 functions computed in
    // double (about 40 instructions each) and also loads a buffer at an
    // index that varies by element leaves each group's loads exposed behind
    // that work: two groups a lane overlap them (map_unroll_gx=0: one).
    // Config 5's adjoint map (exp of the path, and the terminal price
    // gathered for the gather's adjoint computed in place): 528 -> 426 us;
    // its maps that only stream measured slower with two groups (325 ->
    // 360 us), as did the f32 Horner map above.
    int64_t UN = tune("map_unroll", -1);
    if (UN < 0) {
      UN = std::count(f.code.begin(), f.code.end(), '\n') >= 48 ? 4 / G : 1;
      if (UN == 1 && G == 4 && tune("map_unroll_gx", 1) && calls_f32_fn(f.code) && varying_load(f.code)) UN = 2;
    }
    UN = std::max<int64_t>(1, std::min<int64_t>(4, UN));
    // A whole-tensor reduction of this output folds it here: each lane
    // folds the elements it stores, each wave combines its lanes and stores
    // one partial and whether it held any element (the last workgroup's
    // waves may hold none), and the reduction's root folds the partials.
    // Its input is then never read back (config 1: s = sum(r) over 2^24).
    // No workgroup barrier: waves leave as they finish.
    std::string rc, ri, TR = T;
    int part = -1, pflag = -1;
    if (fuse) {
      const TNode &rn = g.ts[fr->second];
      rc = "c_" + std::to_string(rn.id);
      ri = "z_" + std::to_string(rn.id);
      TR = dt_ctype(rn.dt);
      src << gen.combine_fn(rc, rn.body, rn.dt) << gen.const_fn(ri, rn.init, rn.dt);
      const int64_t np = 4 * std::min<int64_t>(cdiv(std::max<int64_t>(1, N / G), 256 * UN), tune("map_blocks", 1 << 22));
      part = add_buf("t" + std::to_string(rn.id) + "_partials", rn.dt, np, BufRole::Scratch);
      pflag = add_buf("t" + std::to_string(rn.id) + "_partial_has", DT::I32, np, BufRole::Scratch);
      free_after[part] = fr->second;
      free_after[pflag] = fr->second;
      fused_part_of_red[fr->second] = {part, pflag, np};
      p.out.push_back(part);
      p.out.push_back(pflag);
      args.clear();
      params = param_list(p, args);
    }
    static const char *comp[] = {"x", "y", "z", "w"};
    // the value folded for element u of the group at i held in rv: the
    // output's own, or the reduction's expression over it and the loads
    auto fold_val = [&](const std::string &i, const std::string &rv, int u) {
      if (!fexpr) return rv + "." + comp[u];
      const std::string idx = u == 0 ? i : "(" + i + " + " + std::to_string(u) + ")";
      return fe.call(idx, [&](int b) { return (b == out ? rv : "l" + std::to_string(b)) + "." + comp[u]; });
    };
    // Each workgroup takes a contiguous run of 256 * UN groups, lane l its
    // groups l, l + 256, ..., and the grid covers the whole tensor, so each
    // lane makes one pass. Resident waves then touch one contiguous window
    // of HBM. A capped grid whose lanes stride by the grid's width keeps
    // several windows open at once, a quarter of the tensor apart, and
    // loses DRAM row locality: 2^28 f32 saxpy at 65536 workgroups 568 us,
    // at one group a lane 506 us (5.67 -> 6.38 TB/s).
    std::ostringstream k;
    k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "(" << params << ") {\n"
      << "  const int stride = gridDim.x * " << 256 * UN << ";\n"
      << "  const int nvec = " << N / G << ";\n";
    if (fuse) k << "  " << TR << " acc = " << ri << "();\n  bool has = false;\n";
    if (UN == 1) {
      k << "  for (int v = blockIdx.x * 256 + threadIdx.x; v < nvec; v += stride) {\n"
        << "    const int i = v * " << G << ";\n"
        << vec_loads(f, "i", "    ", tyof(), ntl, G) << (fexpr ? vec_loads(fx, "i", "    ", tyof(), ntl, G) : "")
        << "    " << VG << "<" << T << "> r;\n";
      for (int u = 0; u < G; u++) k << "    r." << comp[u] << " = " << lane_call(f, "i", u) << ";\n";
      if (store && nts)
        k << "    cc_st" << G << "_nt(b" << out << " + i, r);\n";
      else if (store)
        k << "    *(" << VG << "<" << T << ">*)(b" << out << " + i) = r;\n";
      if (side >= 0)
        for (int u = 0; u < G; u++)
          k << "    " << side_st("i + " + std::to_string(u), std::string("r.") + comp[u]) << "\n";
      if (fuse)
        for (int u = 0; u < G; u++) k << "    " << fold_in(rc, TR, fold_val("i", "r", u)) << "\n";
    } else {
      k << "  for (int v0 = blockIdx.x * " << 256 * UN << " + threadIdx.x; v0 < nvec; v0 += stride) {\n"
        << "    " << VG << "<" << T << "> r[" << UN << "];\n";
      for (int64_t q = 0; q < UN; q++) {
        k << "    {\n"
          << "      const int i = min(v0 + " << q * 256 << ", nvec - 1) * " << G << ";\n"
          << vec_loads(f, "i", "      ", tyof(), ntl, G) << (fexpr ? vec_loads(fx, "i", "      ", tyof(), ntl, G) : "");
        for (int u = 0; u < G; u++) k << "      r[" << q << "]." << comp[u] << " = " << lane_call(f, "i", u) << ";\n";
        // an expression's loads live in this block: folded here, in the
        // same order (a clamped group is its owner's: folded once)
        if (fexpr)
          for (int u = 0; u < G; u++)
            k << "      "
              << fold_in_if(rc, TR, fold_val("i", "r[" + std::to_string(q) + "]", u),
                            "v0 + " + std::to_string(q * 256) + " < nvec")
              << "\n";
        k << "    }\n";
      }
      for (int64_t q = 0; q < UN; q++) {
        std::string iq = "min(v0 + " + std::to_string(q * 256) + ", nvec - 1) * " + std::to_string(G);
        if (store && nts)
          k << "    cc_st" << G << "_nt(b" << out << " + " << iq << ", r[" << q << "]);\n";
        else if (store)
          k << "    *(" << VG << "<" << T << ">*)(b" << out << " + " << iq << ") = r[" << q << "];\n";
        // a clamped group stores its owner's values again, here as there
        if (side >= 0)
          for (int u = 0; u < G; u++)
            k << "    " << side_st(iq + " + " + std::to_string(u), "r[" + std::to_string(q) + "]." + comp[u]) << "\n";
      }
      // a clamped group is its owner's: folded once, by the owner
      if (fuse && !fexpr)
        for (int64_t q = 0; q < UN; q++)
          for (int u = 0; u < G; u++)
            k << "    " << fold_in_if(rc, TR, "r[" + std::to_string(q) + "]." + comp[u], "v0 + " + std::to_string(q * 256) + " < nvec")
              << "\n";
    }
    k << "  }\n"
      << "  for (int i = nvec * " << G << " + blockIdx.x * 256 + threadIdx.x; i < " << N << "; i += gridDim.x * 256)";
    if (fuse || side >= 0)
      k << " {\n    const " << T << " v_ = " << f.call_scalar("i") << ";\n    "
        << (store ? "b" + std::to_string(out) + "[i] = v_;\n    " : std::string())
        << (fuse ? fold_in(rc, TR,
                           fexpr ? fe.call("i", [&](int b) { return b == out ? std::string("v_")
                                                                             : "b" + std::to_string(b) + "[i]"; })
                                 : std::string("v_"))
                 : std::string())
        << (side >= 0 ? side_st("i", "v_") : std::string())
        << "\n  }\n";
    else
      k << "\n    b" << out << "[i] = " << f.call_scalar("i") << ";\n";
    if (fuse)
      k << "  for (int off = 32; off > 0; off >>= 1) " << xor_combine(rc, TR, "off") << "\n"
        << "  if ((threadIdx.x & 63) == 0) {\n"
        << "    const int w = blockIdx.x * 4 + (threadIdx.x >> 6);\n"
        << "    b" << part << "[w] = acc;\n"
        << "    b" << pflag << "[w] = has;\n"
        << "  }\n";
    k << "}\n";
    src << k.str();
    int64_t nvec = std::max<int64_t>(1, N / G);
    int grid = (int)std::min<int64_t>(cdiv(nvec, 256 * UN), tune("map_blocks", 1 << 22));
    if (fexpr) map_extra_moved[t] = fn_bytes(fx, N);
    return {add_kernel(kname, args, grid, 256, "map")};
  }

  // ---- Row-sequential reduce/scan ----------------------------------------
  // With enough rows, one lane owns one row and folds it strictly left to
  // right from init, in exactly the interpreter's order (R2), so f32 sums
  // and prefix sums are bit-identical to it. Workgroups stage R rows x W
  // columns through LDS with coalesced (4-wide) global accesses; the next
  // tile's loads are in flight in registers while the lanes fold the
  // current one. Used when rows >= 1024, where there are enough lanes to
  // keep HBM busy.
  std::vector<int> lower_rows_seq(int t, bool scan, const ElemFn &f, const std::string &cmb, const std::string &ini,
                                  int64_t rows, int64_t len) {
    const TNode &n = g.ts[t];
    std::string kname = "k_" + std::to_string(n.id);
    std::string T = dt_ctype(n.dt);
    int out = buf_of[t];
    // LDS bytes per tile and the fewest workgroups to aim for; reductions
    // (no stores) and scans measure best at different points.
    int64_t elems = (scan ? tune("rs_bytes", 32768) : tune("rr_bytes", 65536)) / dt_size(n.dt);
    int64_t min_groups = scan ? tune("rs_groups", 256) : tune("rr_groups", 256);
    int64_t R = 1;
    while (R < 64 && rows / (R * 2) >= min_groups) R *= 2;
    int64_t W = std::min<int64_t>(elems / R, std::max<int64_t>(4, pow2ceil(len)));
    elems = R * W;
    int64_t E = cdiv(elems, 1024);  // 4-element groups per thread
    int64_t NT = cdiv(len, W);
    int64_t REM = len - (NT - 1) * W;
    int64_t S = W + 4;               // row stride keeps 4-element groups 16-byte aligned
    // Elements per batch of LDS reads in the fold: a multiple of 4 that
    // divides W, so a batch never reads past its row.
    // Long scanned rows read 64 at a time; short ones (whose loads carry the
    // heavier element functions, as in Monte Carlo paths) 16.
    int64_t CH = std::max<int64_t>(4, std::min<int64_t>(scan ? tune("rs_chunk", W >= 256 ? 64 : 16) : tune("rr_chunk", 16), W));
    while (CH > 4 && (W % CH || CH % 4)) CH -= 4;
    bool vec = len % 4 == 0;
    // Streaming (non-temporal) accesses, a bit mask: 1 a scan's stores,
    // 2 a reduction's loads, 4 a scan's loads.
    int64_t rs_nt = tune("rs_nt", -1);
    if (rs_nt < 0)  // 8-byte scans stream their stores only
      rs_nt = streams(fn_bytes(f, rows * len) + (scan ? rows * len : rows) * dt_size(n.dt)) ? (narrow(f, n.dt) ? 5 : 1) : 0;
    if (n.dt == DT::BOOL) rs_nt = 0;
    for (int b : f.ident)
      if (prog.bufs[b].dt == DT::BOOL) rs_nt &= 1;
    const bool nt_loads = (rs_nt & (scan ? 4 : 2)) != 0, nt_stores = scan && (rs_nt & 1);
    // 8-byte scans store pairs (rs_pairs8=0: 4-element groups)
    const bool pairs8 = tune("rs_pairs8", 1) != 0;
    // a scan's side buffer of row-last elements (Gen::rowlast_), if any
    const auto sd = scan ? gen.rowlast_.find(t) : gen.rowlast_.end();
    const int side = sd != gen.rowlast_.end() ? sd->second.first : -1;
    Params p;
    add_in(p, f);
    p.out.push_back(out);
    if (side >= 0) p.out.push_back(side);
    std::vector<int> args;
    std::string params = param_list(p, args);
    static const char *comp[] = {"x", "y", "z", "w"};
    std::string V4 = "cc_v4<" + T + ">";
    // Tiles in flight in registers while one is folded: D register buffers
    // rotate, buffer d receiving tile kt + 1 + D when tile kt has been folded.
    const int64_t D = std::max<int64_t>(1, std::min<int64_t>(2, scan ? tune("rs_depth", 1) : tune("rr_depth", 1)));
    // Split roles, for rows of four tiles or more: wave 0 folds tile kt
    // from one LDS buffer while four loader waves move tile kt + 1 from
    // registers into the other, load tile kt + 3 (two tiles in flight) and,
    // in scans, store tile kt - 1. Done in turn by one workgroup, the fold
    // and the wait for the next tile add up (the 8192^2 add reduction: 26.7
    // us folding and 13 us waiting and moving per workgroup). Measured on
    // 8192^2 f32: the row scan 101.5 -> 93.5-95.6 us split; the add and
    // max reductions 55 / 49 -> 58 / 54 us, so reductions keep the turns.
    const bool split = tune(scan ? "rs_split" : "rr_split", scan ? 1 : 0) != 0 && NT >= 4 &&
                       2 * R * S * dt_size(n.dt) <= 150 * 1024;
    const int NTH = split ? 320 : 256;
    std::ostringstream k;
    k << "extern \"C\" __global__ __launch_bounds__(" << NTH << ") void " << kname << "(" << params << ") {\n";
    if (split)
      k << "  __shared__ " << V4 << " sm4a[" << R * S / 4 << "], sm4b[" << R * S / 4 << "];\n"
        << "  " << T << "* const sma = (" << T << "*)sm4a;\n"
        << "  " << T << "* const smb = (" << T << "*)sm4b;\n"
        << "  const int lt = (int)threadIdx.x - 64;  // loader index (threads 64..319)\n";
    else
      k << "  __shared__ " << V4 << " sm4[" << R * S / 4 << "];\n"
        << "  " << T << "* const sm = (" << T << "*)sm4;\n";
    for (int64_t d = 0; d < (split ? 2 : D); d++) k << "  " << T << " rg" << d << "[" << E * 4 << "];\n";
    k << "  for (int g0 = blockIdx.x * " << R << "; g0 < " << rows << "; g0 += gridDim.x * " << R << ") {\n";
    // Tile c0 into registers: group u of thread t covers flat tile elements
    // q..q+3 with q = 4 (t + 256 u), at row q / W, column q % W.
    auto load = [&](const std::string &c0, const std::string &rg, const std::string &tid = "threadIdx.x") {
      std::ostringstream l;
      l << "    {\n"
        << "      const int c0 = " << c0 << ";\n"
        << "#pragma unroll\n"
        << "      for (int u = 0; u < " << E << "; u++) {\n"
        << "        const int q = 4 * (" << tid << " + 256 * u);\n"
        << "        const int rr = q / " << W << ", j = q - rr * " << W << ";\n"
        << "        const int row = min(g0 + rr, " << rows - 1 << ");\n"
        << "        if (q < " << elems << ") {\n";
      // Groups past the last row or column read a valid element instead
      // (row clamped, column 0) and are never consumed: no load sits
      // behind a branch, so a thread's loads are all in flight together.
      if (vec) {
        l << "          const int i = row * " << len << " + (c0 + j < " << len << " ? c0 + j : 0);\n"
          << vec_loads(f, "i", "          ", tyof(), nt_loads);
        for (int c = 0; c < 4; c++) l << "          " << rg << "[4 * u + " << c << "] = " << lane_call(f, "i", c) << ";\n";
      } else {
        for (int c = 0; c < 4; c++)
          l << "          { const int i = row * " << len << " + (c0 + j + " << c << " < " << len << " ? c0 + j + " << c
            << " : 0); " << rg << "[4 * u + " << c << "] = " << f.call_scalar("i") << "; }\n";
      }
      l << "        }\n"
        << "      }\n"
        << "    }\n";
      return l.str();
    };
    auto to_lds = [&](const std::string &rg, const std::string &tid = "threadIdx.x", const std::string &buf = "sm4") {
      std::ostringstream l;
      l << "#pragma unroll\n"
        << "    for (int u = 0; u < " << E << "; u++) {\n"
        << "      const int q = 4 * (" << tid << " + 256 * u);\n"
        << "      const int rr = q / " << W << ", j = q - rr * " << W << ";\n"
        << "      if (q < " << elems << ") {\n"
        << "        " << V4 << " w;\n";
      for (int c = 0; c < 4; c++) l << "        w." << comp[c] << " = " << rg << "[4 * u + " << c << "];\n";
      l << "        " << buf << "[(rr * " << S << " + j) / 4] = w;\n"
        << "      }\n"
        << "    }\n";
      return l.str();
    };
    // Lane r folds row r of tile kt, held in LDS at `smp` (scans write the
    // prefixes back in place).
    auto fold_tile = [&](const std::string &smp) {
      std::ostringstream b;
      b << "      if (threadIdx.x < " << R << " && g0 + threadIdx.x < " << rows << ") {\n"
        << "        " << T << "* const s = " << smp << " + threadIdx.x * " << S << ";\n"
        << "        if (kt + 1 < " << NT << " || " << REM << " == " << W << ") {\n"
        << "          for (int j0 = 0; j0 < " << W << "; j0 += " << CH << ") {\n"
        << "            " << T << " tv[" << CH << "];\n"
        << "#pragma unroll\n"
        << "            for (int u = 0; u < " << CH / 4 << "; u++) {\n"
        << "              const " << V4 << " w = ((const " << V4 << "*)(s + j0))[u];\n"
        << "              tv[4 * u] = w.x; tv[4 * u + 1] = w.y; tv[4 * u + 2] = w.z; tv[4 * u + 3] = w.w;\n"
        << "            }\n"
        << "#pragma unroll\n"
        << "            for (int u = 0; u < " << CH << "; u++) { acc = " << cmb << "(acc, tv[u]);"
        << (scan ? " tv[u] = acc;" : "") << " }\n";
      if (scan)
        b << "#pragma unroll\n"
          << "            for (int u = 0; u < " << CH / 4 << "; u++) {\n"
          << "              " << V4 << " w; w.x = tv[4 * u]; w.y = tv[4 * u + 1]; w.z = tv[4 * u + 2]; w.w = tv[4 * u + 3];\n"
          << "              ((" << V4 << "*)(s + j0))[u] = w;\n"
          << "            }\n";
      b << "          }\n"
        << "        } else {\n"
        << "          for (int j = 0; j < " << REM << "; j++) { acc = " << cmb << "(acc, s[j]);"
        << (scan ? " s[j] = acc;" : "") << " }\n"
        << "        }\n"
        << "      }\n";
      return b.str();
    };
    // A scan's store of tile `ktx` from the LDS buffer `buf`, thread `tid`
    // taking the same groups it moved into LDS. `own` where the thread then
    // refills those LDS words with no barrier between (the split roles'
    // loaders): it must read only the words it writes next, so the 8-byte
    // pairs, which another thread's groups hold, are not used there.
    auto store_tile = [&](const std::string &ktx, const std::string &tid, const std::string &buf, bool own = false) {
      std::ostringstream b;
      if (vec && dt_size(n.dt) == 8 && pairs8 && !own) {
        // 8-byte values in pairs: one 16-byte access a lane, consecutive
        // lanes at consecutive addresses, so each store instruction writes
        // whole lines (a 4-element group of 8-byte values is two 16-byte
        // accesses 32 bytes apart, half-line writes in each instruction)
        const std::string V2 = "cc_v2<" + T + ">";
        // pair u of a lane lies 512 u elements past pair 0, 512 / W rows
        // further down in the same column where W divides 512
        const bool rows_step = 512 % W == 0;
        b << "      {\n"
          << "      const int q0_ = 2 * (int)(" << tid << "), rr0_ = q0_ / " << W << ", j0_ = q0_ - rr0_ * " << W << ";\n"
          << "#pragma unroll\n"
          << "      for (int u = 0; u < " << 2 * E << "; u++) {\n"
          << "        const int c0 = (" << ktx << ") * " << W << ";\n"
          << "        const int q = q0_ + 512 * u;\n";
        if (rows_step)
          b << "        const int rr = rr0_ + " << 512 / W << " * u, j = j0_;\n";
        else
          b << "        const int rr = q / " << W << ", j = q - rr * " << W << ";\n";
        b << "        const int row = g0 + rr;\n"
          << "        if (q < " << elems << " && row < " << rows << ") {\n"
          << "          const int i = row * " << len << " + c0 + j;\n"
          << "          const " << V2 << " o = ((const " << V2 << "*)" << buf << ")[(rr * " << S << " + j) / 2];\n";
        if (nt_stores)
          b << "          if (c0 + j < " << len << ") cc_st2_nt(b" << out << " + i, o);\n";
        else
          b << "          if (c0 + j < " << len << ") *(" << V2 << "*)(b" << out << " + i) = o;\n";
        b << "        }\n"
          << "      }\n"
          << "      }\n";
        return b.str();
      }
      b << "#pragma unroll\n"
        << "      for (int u = 0; u < " << E << "; u++) {\n"
        << "        const int c0 = (" << ktx << ") * " << W << ";\n"
        << "        const int q = 4 * (" << tid << " + 256 * u);\n"
        << "        const int rr = q / " << W << ", j = q - rr * " << W << ";\n"
        << "        const int row = g0 + rr;\n"
        << "        if (q < " << elems << " && row < " << rows << ") {\n"
        << "          const int i = row * " << len << " + c0 + j;\n"
        << "          const " << V4 << " o = " << buf << "[(rr * " << S << " + j) / 4];\n";
      if (vec) {
        if (nt_stores)
          b << "          if (c0 + j < " << len << ") cc_st4_nt(b" << out << " + i, o);\n";
        else
          b << "          if (c0 + j < " << len << ") *(" << V4 << "*)(b" << out << " + i) = o;\n";
      } else {
        for (int c = 0; c < 4; c++)
          b << "          if (c0 + j + " << c << " < " << len << ") b" << out << "[i + " << c << "] = o." << comp[c]
            << ";\n";
      }
      b << "        }\n"
        << "      }\n";
      return b.str();
    };
    // One tile: fold it, store it (scans), move the next tile from
    // registers into LDS, refill the registers.
    auto body = [&](const std::string &rg) {
      std::ostringstream b;
      b << fold_tile("sm") << "      __syncthreads();\n";
      if (scan) b << store_tile("kt", "threadIdx.x", "sm4") << "      __syncthreads();\n";
      b << "      if (kt + 1 < " << NT << ") {\n" << to_lds(rg) << "      }\n"
        << "      if (kt + " << 1 + D << " < " << NT << ") {\n"
        << load("(kt + " + std::to_string(1 + D) + ") * " + std::to_string(W), rg) << "      }\n"
        << "      __syncthreads();\n";
      return b.str();
    };
    if (split) {
      // Tile kt sits in buffer kt & 1; registers rg(kt & 1) hold tile
      // kt + 1 while tile kt is folded.
      auto step = [&](int d) {
        const std::string mine = d ? "smb" : "sma", other4 = d ? "sm4a" : "sm4b", rg = "rg" + std::to_string(d);
        std::ostringstream b;
        b << fold_tile(mine) << "      if (threadIdx.x >= 64) {\n";
        if (scan) b << "      if (kt >= 1) {\n" << store_tile("kt - 1", "lt", other4, true) << "      }\n";
        b << "      if (kt + 1 < " << NT << ") {\n" << to_lds(rg, "lt", other4) << "      }\n"
          << "      if (kt + 3 < " << NT << ") {\n"
          << load("(kt + 3) * " + std::to_string(W), rg, "lt") << "      }\n"
          << "      }\n"
          << "      __syncthreads();\n";
        return b.str();
      };
      k << "    if (threadIdx.x >= 64) {\n"
        << load("0", "rg0", "lt") << to_lds("rg0", "lt", "sm4a") << load(std::to_string(W), "rg0", "lt")
        << load(std::to_string(2 * W), "rg1", "lt") << "    }\n"
        << "    __syncthreads();\n"
        << "    " << T << " acc = " << ini << "();\n"
        << "    for (int kt0 = 0; kt0 < " << NT << "; kt0 += 2) {\n"
        << "      {\n      const int kt = kt0;\n" << step(0) << "      }\n"
        << "      if (kt0 + 1 < " << NT << ") {\n      const int kt = kt0 + 1;\n" << step(1) << "      }\n"
        << "    }\n";
      if (scan && side >= 0)
        k << "    if (threadIdx.x < " << R << " && g0 + threadIdx.x < " << rows << ") b" << side
          << "[g0 + threadIdx.x] = acc;\n";
      if (scan)
        k << "    if (threadIdx.x >= 64) {\n" << store_tile(std::to_string(NT - 1), "lt", (NT - 1) % 2 ? "sm4b" : "sm4a")
          << "    }\n"
          << "    __syncthreads();\n";
      else
        k << "    if (threadIdx.x < " << R << " && g0 + threadIdx.x < " << rows << ") b" << out
          << "[g0 + threadIdx.x] = acc;\n";
      k << "  }\n}\n";
      src << k.str();
      int grid = (int)std::min<int64_t>(cdiv(rows, R), 1 << 20);
      return {add_kernel(kname, args, grid, NTH, scan ? "scan_rowseq" : "reduce_rowseq")};
    }
    k << load("0", "rg0") << to_lds("rg0");
    for (int64_t d = 0; d < D; d++)
      k << "    if (" << NT << " > " << d + 1 << ") {\n"
        << load(std::to_string((d + 1) * W), "rg" + std::to_string(d)) << "    }\n";
    k << "    __syncthreads();\n"
      << "    " << T << " acc = " << ini << "();\n"
      << "    for (int kt0 = 0; kt0 < " << NT << "; kt0 += " << D << ") {\n";
    for (int64_t d = 0; d < D; d++) {
      k << "      if (kt0 + " << d << " < " << NT << ") {\n"
        << "      const int kt = kt0 + " << d << ";\n"
        << body("rg" + std::to_string(d)) << "      }\n";
    }
    k << "    }\n";
    if (!scan || side >= 0)
      k << "    if (threadIdx.x < " << R << " && g0 + threadIdx.x < " << rows << ") b" << (scan ? side : out)
        << "[g0 + threadIdx.x] = acc;\n";
    k << "  }\n}\n";
    src << k.str();
    int grid = (int)std::min<int64_t>(cdiv(rows, R), 1 << 20);
    return {add_kernel(kname, args, grid, 256, scan ? "scan_rowseq" : "reduce_rowseq")};
  }

  // ---- Reduce root (K2-K4 -> wave / block / split-row reductions) --------
  // Whether the combine (x0, x1) -> body is op(x0, x1) or op(x1, x0) for
  // an op that may be folded in any grouping: with floats too, one whose
  // result depends on the grouping only through rounding (add, mul).
  bool any_order(int body, DT dt, bool floats) const {
    const XNode &x = g.xs[body];
    if (x.kind != XK::Bin || x.a < 0 || x.b < 0) return false;
    const XNode &l = g.xs[x.a], &r = g.xs[x.b];
    if (l.kind != XK::Arg || r.kind != XK::Arg || l.arg == r.arg) return false;
    if (x.op == B_MIN || x.op == B_MAX) return true;
    const bool integer = dt == DT::I32 || dt == DT::I64;
    if (!integer) return floats && (x.op == B_ADD || x.op == B_MUL);
    return x.op == B_ADD || x.op == B_MUL || x.op == B_AND || x.op == B_OR || x.op == B_XOR;
  }

  std::vector<int> lower_reduce(int t) {
    const TNode &n = g.ts[t];
    const TNode &s = g.ts[n.a];
    std::string id = std::to_string(n.id);
    std::string kname = "k_" + id;
    std::string T = dt_ctype(n.dt);
    int out = buf_of[t];
    int64_t len = row_length(s.shape);
    int64_t rows = n.numel;
    std::string cmb = "c_" + id, ini = "z_" + id;
    const auto fp = fused_part_of_red.find(t);
    if (fp != fused_part_of_red.end()) {
      // The map that wrote the input left one partial a wave (its kernel
      // emitted the combine): fold them, 1024 a workgroup in a first kernel
      // where there are more, then the rest and init once.
      std::vector<int> ks;
      const int in = fp->second.part, flags = fp->second.flags;
      const int64_t np = fp->second.count;
      // the flags matter in the first fold only: a run of 1024 partials
      // starts at a workgroup's first wave, which is never empty
      // Each workgroup folds runs of 1024 partials, four a lane loaded
      // together (indices clamped into the run, so no load waits behind a
      // branch), then its lanes.
      auto fold_kernel = [&](const std::string &name, int from, int to, int64_t count, int64_t per, bool final) {
        const bool flagged = from == in;
        Params p;
        p.in.push_back(from);
        if (flagged) p.in.push_back(flags);
        p.out.push_back(to);
        std::vector<int> args;
        std::string params = param_list(p, args);
        const std::string P = "b" + std::to_string(from), F = "b" + std::to_string(flags);
        std::ostringstream k;
        k << "extern \"C\" __global__ __launch_bounds__(256) void " << name << "(" << params << ") {\n"
          << "  __shared__ " << T << " wpart[4];\n"
          << "  __shared__ bool whas[4];\n"
          << "  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;\n"
          << "  const int lo = blockIdx.x * " << per << ", hi = min(lo + " << per << ", " << count << ");\n"
          << "  " << T << " acc = " << ini << "();\n"
          << "  bool has = false;\n"
          << "  for (int c0 = lo; c0 < hi; c0 += 1024) {\n"
          << "    " << T << " v[4];\n"
          << "    bool ok[4];\n"
          << "#pragma unroll\n"
          << "    for (int u = 0; u < 4; u++) {\n"
          << "      const int q = c0 + (int)threadIdx.x + 256 * u, qc = min(q, hi - 1);\n"
          << "      v[u] = " << P << "[qc];\n"
          << "      ok[u] = q < hi" << (flagged ? " && " + F + "[qc] != 0" : "") << ";\n"
          << "    }\n"
          << "#pragma unroll\n"
          << "    for (int u = 0; u < 4; u++) " << fold_in_if(cmb, T, "v[u]", "ok[u]") << "\n"
          << "  }\n"
          << "  for (int off = 32; off > 0; off >>= 1) " << xor_combine(cmb, T, "off") << "\n"
          << "  if (lane == 0) { wpart[wid] = acc; whas[wid] = has; }\n"
          << "  __syncthreads();\n"
          << "  if (threadIdx.x == 0) {\n"
          << "    " << T << " t = " << ini << "();\n    bool th = false;\n"
          << "    for (int w = 0; w < 4; w++) if (whas[w]) { t = th ? " << cmb << "(t, wpart[w]) : wpart[w]; th = true; }\n"
          << "    b" << to << "[blockIdx.x] = " << (final ? cmb + "(" + ini + "(), t)" : "t") << ";\n"
          << "  }\n"
          << "}\n";
        src << k.str();
        ks.push_back(add_kernel(name, args, (int)cdiv(count, per), 256, "reduce_split_fold"));
      };
      // Up to fold_one partials (16384; 0: never) fold in one workgroup of
      // 1024 threads instead of two kernels: thread t folds partials t,
      // t + 1024, ... in that order, sixteen loads in flight at a time,
      // then the waves fold by butterfly and thread 0 folds the 16 waves in
      // order and applies init once. A small kernel costs a few
      // microseconds whatever it moves, so the second one is what goes: the
      // S20 Greeks step (three sums of 16384 partials) 0.105 -> 0.100 ms.
      // Past that, one workgroup's share of the loads costs what the
      // second kernel saves (f64 S20, 32768 partials: 0.154 -> 0.160 ms;
      // config 1, 65536: no change).
      const int64_t one = tune("fold_one", 16384);
      if (np > 1024 && np <= one) {
        Params p;
        p.in.push_back(in);
        p.in.push_back(flags);
        p.out.push_back(out);
        std::vector<int> args;
        std::string params = param_list(p, args);
        const int64_t K = cdiv(np, 1024), CH = std::min<int64_t>(16, K);
        const std::string P = "b" + std::to_string(in), F = "b" + std::to_string(flags);
        std::ostringstream k;
        k << "extern \"C\" __global__ __launch_bounds__(1024) void " << kname << "(" << params << ") {\n"
          << "  __shared__ " << T << " wpart[16];\n"
          << "  __shared__ bool whas[16];\n"
          << "  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;\n"
          << "  " << T << " acc = " << ini << "();\n"
          << "  bool has = false;\n"
          << "  for (int u0 = 0; u0 < " << K << "; u0 += " << CH << ") {\n"
          << "    " << T << " v[" << CH << "];\n"
          << "    bool ok[" << CH << "];\n"
          << "#pragma unroll\n"
          << "    for (int u = 0; u < " << CH << "; u++) {\n"
          << "      const int q = (int)threadIdx.x + 1024 * (u0 + u), qc = min(q, " << np - 1 << ");\n"
          << "      v[u] = " << P << "[qc];\n"
          << "      ok[u] = q < " << np << " && " << F << "[qc] != 0;\n"
          << "    }\n"
          << "#pragma unroll\n"
          << "    for (int u = 0; u < " << CH << "; u++) " << fold_in_if(cmb, T, "v[u]", "ok[u]") << "\n"
          << "  }\n"
          << "  for (int off = 32; off > 0; off >>= 1) " << xor_combine(cmb, T, "off") << "\n"
          << "  if (lane == 0) { wpart[wid] = acc; whas[wid] = has; }\n"
          << "  __syncthreads();\n"
          << "  if (threadIdx.x == 0) {\n"
          << "    " << T << " t = " << ini << "();\n"
          << "    bool th = false;\n"
          << "    for (int w = 0; w < 16; w++) if (whas[w]) { t = th ? " << cmb << "(t, wpart[w]) : wpart[w]; th = true; }\n"
          << "    b" << out << "[0] = " << cmb << "(" << ini << "(), t);\n"
          << "  }\n"
          << "}\n";
        src << k.str();
        ks.push_back(add_kernel(kname, args, 1, 1024, "reduce_split_fold"));
      } else if (np > 1024) {
        const int64_t n1 = cdiv(np, 1024);
        int mid = add_buf("t" + id + "_partials2", n.dt, n1, BufRole::Scratch);
        fold_kernel(kname + "_fold", in, mid, np, 1024, false);
        fold_kernel(kname, mid, out, n1, n1, true);
      } else {
        fold_kernel(kname, in, out, np, np, true);
      }
      return ks;
    }
    src << gen.combine_fn(cmb, n.body, n.dt) << gen.const_fn(ini, n.init, n.dt);
    if (rows == 0) return {};
    if (len == 0) {
      // Every row is empty: the output is init (R2).
      Params p;
      p.out.push_back(out);
      std::vector<int> args;
      std::string params = param_list(p, args);
      src << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "(" << params << ") {\n"
          << "  for (int r = blockIdx.x * 256 + threadIdx.x; r < " << rows << "; r += gridDim.x * 256) b" << out
          << "[r] = " << ini << "();\n}\n";
      return {add_kernel(kname, args, (int)std::min<int64_t>(cdiv(rows, 256), 4096), 256, "reduce_empty")};
    }
    ElemFn f = gen.element_fn("f_" + id, n.a, false, true);
    src << f.code;
    // 1024 rows or more fold one lane a row, in order, unless the rows are
    // long (rr_tree_len) and the combine allows any grouping: max and min
    // (which propagate NaN and order -0 below +0), wrapping integer add,
    // mul and bit operations, all bit-exact in any grouping; and float add
    // and mul, whose tree differs from the in-order fold by rounding only.
    // Those fold as a tree, a workgroup or a wave a row. A GiB of f32 or
    // i32 rows, µs in order against as a tree: 8192 long 205-221 / 155,
    // 2048 long 188-191 / 178, 1000 long 172-176 / 174, 256 long 184-190 /
    // 198, 64 long 181 / 425. rr_tree=1 folds float rows in order
    // (bit-identical to the interpreter), rr_tree=0 every row.
    const int64_t tree = tune("rr_tree", 2);
    const bool as_tree = tree >= 1 && len >= tune("rr_tree_len", 1024) && any_order(n.body, n.dt, tree >= 2);
    if (rows >= 1024 && !as_tree) return lower_rows_seq(t, false, f, cmb, ini, rows, len);
    bool vec = len % 4 == 0;
    if (len <= 2048) {
      // One wave (or a power-of-two segment of one) per row.
      int64_t S = std::min<int64_t>(64, pow2ceil(len));
      int64_t rpw = 64 / S;
      Params p;
      add_in(p, f);
      p.out.push_back(out);
      std::vector<int> args;
      std::string params = param_list(p, args);
      std::ostringstream k;
      k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "(" << params << ") {\n"
        << "  const int lane = threadIdx.x & 63;\n"
        << "  const int seg = lane / " << S << ";\n"
        << "  const int sl = lane - seg * " << S << ";\n"
        << "  const int wave = (blockIdx.x * 256 + threadIdx.x) >> 6;\n"
        << "  const int nwaves = gridDim.x * 4;\n"
        << "  for (int rb = wave * " << rpw << "; rb < " << rows << "; rb += nwaves * " << rpw << ") {\n"
        << "    const int r = rb + seg;\n"
        << "    " << T << " acc = " << ini << "();\n"
        << "    bool has = false;\n"
        << "    if (r < " << rows << ") {\n"
        << "      for (int j0 = sl; j0 < " << len << "; j0 += " << 4 * S << ") {\n"
        << "        " << T << " xs[4];\n"
        << "#pragma unroll\n"
        << "        for (int u = 0; u < 4; u++) {\n"
        << "          const int i = r * " << len << " + (j0 + u * " << S << " < " << len << " ? j0 + u * " << S
        << " : j0);\n"
        << "          xs[u] = " << f.call_scalar("i") << ";\n"
        << "        }\n"
        << "#pragma unroll\n"
        << "        for (int u = 0; u < 4; u++) "
        << fold_in_if(cmb, T, "xs[u]", "j0 + u * " + std::to_string(S) + " < " + std::to_string(len)) << "\n"
        << "      }\n"
        << "    }\n";
      for (int64_t off = S / 2; off > 0; off /= 2) k << "    " << xor_combine(cmb, T, std::to_string(off)) << "\n";
      k << "    if (r < " << rows << " && sl == 0) b" << out << "[r] = has ? " << cmb << "(" << ini << "(), acc) : " << ini
        << "();\n"
        << "  }\n}\n";
      src << k.str();
      int64_t waves = cdiv(rows, rpw);
      int grid = (int)std::min<int64_t>(cdiv(waves, 4), 16384);
      return {add_kernel(kname, args, grid, 256, "reduce_wave")};
    }
    // Accumulators carry an empty flag, so init is applied exactly once, to
    // the row's total (init is not assumed to be the combine's identity).
    std::string block_reduce = "    for (int off = 32; off > 0; off >>= 1) " + xor_combine(cmb, T, "off") +
                               "\n"
                               "    if (lane == 0) { wpart[wid] = acc; whas[wid] = has; }\n"
                               "    __syncthreads();\n";
    std::string wave_parts = "      " + T + " t = " + ini + "();\n      bool th = false;\n"
                             "      for (int w = 0; w < 4; w++) if (whas[w]) { t = th ? " + cmb +
                             "(t, wpart[w]) : wpart[w]; th = true; }\n";
    // Four strides per iteration, all loads issued before any is folded
    // (a one-load loop leaves each workgroup waiting out one memory latency
    // per stride); strides past the end load at the iteration's first
    // (valid) index and are not folded.
    int64_t red_nt = tune("red_nt", -1);
    if (red_nt < 0) red_nt = narrow(f, n.dt) && streams(fn_bytes(f, rows * len)) ? 1 : 0;
    for (int b : f.ident)
      if (prog.bufs[b].dt == DT::BOOL) red_nt = 0;
    // The column index is 64-bit where a step past the row's end would
    // leave the int range (rows up to 2^31 - 1 long).
    auto fold_loop = [&](const std::string &lo, const std::string &hi) {
      std::ostringstream l;
      const std::string J = len + 2 * 4096 > INT32_MAX ? "long long" : "int";
      if (vec) {
        l << "    for (" << J << " j0 = " << lo << " + threadIdx.x * 4; j0 < " << hi << "; j0 += 4096) {\n";
        for (int b : f.ident) l << "      cc_v4<" << ty(b) << "> l" << b << "_[4];\n";
        l << "#pragma unroll\n"
          << "      for (int u = 0; u < 4; u++) {\n"
          << "        const int i = base + (int)(j0 + u * 1024 < " << hi << " ? j0 + u * 1024 : j0);\n";
        for (int b : f.ident) {
          if (red_nt)
            l << "        l" << b << "_[u] = cc_ld4_nt(b" << b << " + i);\n";
          else
            l << "        l" << b << "_[u] = *(const cc_v4<" << ty(b) << ">*)(b" << b << " + i);\n";
        }
        l << "      }\n"
          << "#pragma unroll\n"
          << "      for (int u = 0; u < 4; u++) {\n"
          << "        const bool in = j0 + u * 1024 < " << hi << ";\n"
          << "        const int i = base + (int)(in ? j0 + u * 1024 : j0);\n";
        for (int b : f.ident) l << "        const cc_v4<" << ty(b) << "> l" << b << " = l" << b << "_[u];\n";
        for (int u = 0; u < 4; u++) l << "        " << fold_in_if(cmb, T, lane_call(f, "i", u), "in") << "\n";
        l << "      }\n"
          << "    }\n";
      } else {
        l << "    for (" << J << " j0 = " << lo << " + threadIdx.x; j0 < " << hi << "; j0 += 1024) {\n"
          << "      " << T << " xs[4];\n"
          << "#pragma unroll\n"
          << "      for (int u = 0; u < 4; u++) {\n"
          << "        const int i = base + (int)(j0 + u * 256 < " << hi << " ? j0 + u * 256 : j0);\n"
          << "        xs[u] = " << f.call_scalar("i") << ";\n"
          << "      }\n"
          << "#pragma unroll\n"
          << "      for (int u = 0; u < 4; u++) " << fold_in_if(cmb, T, "xs[u]", "j0 + u * 256 < " + hi) << "\n"
          << "    }\n";
      }
      return l.str();
    };
    if (rows >= 512) {
      // One workgroup per row.
      Params p;
      add_in(p, f);
      p.out.push_back(out);
      std::vector<int> args;
      std::string params = param_list(p, args);
      std::ostringstream k;
      k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "(" << params << ") {\n"
        << "  __shared__ " << T << " wpart[4];\n"
        << "  __shared__ bool whas[4];\n"
        << "  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;\n"
        << "  for (int r = blockIdx.x; r < " << rows << "; r += gridDim.x) {\n"
        << "    const int base = r * " << len << ";\n"
        << "    " << T << " acc = " << ini << "();\n"
        << "    bool has = false;\n"
        << fold_loop("0", std::to_string(len)) << block_reduce << "    if (threadIdx.x == 0) {\n"
        << wave_parts
        << "      b" << out << "[r] = th ? " << cmb << "(" << ini << "(), t) : " << ini << "();\n"
        << "    }\n"
        << "    __syncthreads();\n"
        << "  }\n}\n";
      src << k.str();
      int grid = (int)std::min<int64_t>(rows, 1 << 20);
      return {add_kernel(kname, args, grid, 256, "reduce_block")};
    }
    // Few long rows: split each row over G workgroups that store one partial
    // each; a second kernel folds each row's G partials in order. The kernel
    // boundary makes the partials visible: no per-workgroup release (on a
    // multi-XCD device an agent-scope release writes back the L2) and no
    // counter to reset.
    int64_t unit = vec ? 4096 : 1024;
    int64_t G = std::max<int64_t>(1, std::min<int64_t>(cdiv(2048, rows), cdiv(len, 4096)));
    int64_t chunk = cdiv(cdiv(len, G), unit) * unit;
    G = cdiv(len, chunk);
    int part = add_buf("t" + id + "_partials", n.dt, rows * G, BufRole::Scratch);
    std::vector<int> ks;
    {
      Params p;
      add_in(p, f);
      p.out.push_back(part);
      std::vector<int> args;
      std::string params = param_list(p, args);
      std::ostringstream k;
      k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "_part(" << params << ") {\n"
        << "  __shared__ " << T << " wpart[4];\n"
        << "  __shared__ bool whas[4];\n"
        << "  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;\n"
        << "  const int r = blockIdx.x / " << G << ";\n"
        << "  const int g = blockIdx.x - r * " << G << ";\n"
        << "  const int base = r * " << len << ";\n"
        << "  const int lo = g * " << chunk << ";\n"
        << "  const int hi = min(lo + " << chunk << ", " << len << ");\n"
        << "  " << T << " acc = " << ini << "();\n"
        << "  bool has = false;\n"
        << fold_loop("lo", "hi") << block_reduce << "  if (threadIdx.x == 0) {\n"
        << wave_parts  // every chunk is non-empty, so th holds
        << "    b" << part << "[blockIdx.x] = t;\n"
        << "  }\n"
        << "}\n";
      src << k.str();
      ks.push_back(add_kernel(kname + "_part", args, (int)(rows * G), 256, "reduce_split"));
    }
    {
      Params p;
      p.in.push_back(part);
      p.out.push_back(out);
      std::vector<int> args;
      std::string params = param_list(p, args);
      std::ostringstream k;
      k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "(" << params << ") {\n"
        << "  __shared__ " << T << " wpart[4];\n"
        << "  __shared__ bool whas[4];\n"
        << "  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;\n"
        << "  for (int r = blockIdx.x; r < " << rows << "; r += gridDim.x) {\n"
        << "    " << T << " acc = " << ini << "();\n"
        << "    bool has = false;\n"
        << "    for (int q = threadIdx.x; q < " << G << "; q += 256) " << fold_in(cmb, T, "b" + std::to_string(part) + "[r * " + std::to_string(G) + " + q]") << "\n"
        << block_reduce << "    if (threadIdx.x == 0) {\n"
        << wave_parts
        << "      b" << out << "[r] = " << cmb << "(" << ini << "(), t);\n"
        << "    }\n"
        << "    __syncthreads();\n"
        << "  }\n"
        << "}\n";
      src << k.str();
      ks.push_back(add_kernel(kname, args, (int)std::min<int64_t>(rows, 1024), 256, "reduce_split_fold"));
    }
    return ks;
  }

  // ---- Scan root (K5-K8 -> wave / block / decoupled look-back scans) -----
  // The tile templates' shape for a row of `len` elements of `dt`: NW waves
  // a workgroup, U slices of SL = 256 NW elements a tile, tiles per row.
  struct TileShape {
    int64_t NW, U, SL, tile, tpr;
  };
  static TileShape tile_shape(int64_t len, DT dt) {
    const bool wide = dt_size(dt) == 8;
    auto shape = [&](int64_t NW) {
      TileShape s;
      s.NW = NW;
      int64_t Umax = tune(wide ? "lb_slices8" : "lb_slices4", wide ? 8 : (s.NW == 8 ? 13 : 22));
      if (Umax < 1) throw InvalidArgument("CCHIP_TUNE: look-back slices must be >= 1");
      s.SL = 256 * s.NW;
      s.U = std::min<int64_t>(Umax, std::max<int64_t>(1, cdiv(len, s.SL)));
      s.tile = s.SL * s.U;
      s.tpr = cdiv(len, s.tile);
      return s;
    };
    return shape(tune("lb_waves", 8) == 8 ? 8 : 4);
  }

  // Whether a scan root takes the tile template with one tile a row (one
  // workgroup scans a whole row), as lower_scan decides.
  bool scan_is_row_tile(int t) const {
    const TNode &n = g.ts[t];
    const int64_t len = row_length(n.shape);
    if (len <= 64 || n.numel == 0 || n.dt == DT::BOOL) return false;
    const int64_t rows = n.numel / len;
    if (rows >= 1024 &&
        !(tune("rs_tree", 1) && len >= tune("rs_tree_len", 2048) && any_order(n.body, n.dt, true)))
      return false;
    return tile_shape(len, n.dt).tpr == 1;
  }

  // Whether a reduce root folds its rows as a tree (wave, block or split
  // templates), as lower_reduce decides, rather than in order.
  bool reduce_is_tree(int t) const {
    const TNode &n = g.ts[t];
    const int64_t len = row_length(g.ts[n.a].shape);
    if (n.numel == 0 || len == 0 || n.dt == DT::BOOL) return false;
    const int64_t tree = tune("rr_tree", 2);
    const bool as_tree = tree >= 1 && len >= tune("rr_tree_len", 1024) && any_order(n.body, n.dt, tree >= 2);
    return !(n.numel >= 1024 && !as_tree);
  }

  // Groups of sibling row roots (sibling_fuse=0 keeps every root its own
  // kernels). A reduction joins a scan's group when it reads the same
  // tensor node with the same row shape and would fold as a tree anyway:
  // the fused kernel folds each row's elements in a tree of another shape
  // (each lane its elements in order, then the wave, then the waves in
  // order), so max, min and integer results are the same bits and float
  // add and mul differ by rounding only. The group's kernel runs at its
  // first root's place in the plan: every member reads only what the
  // shared tensor reads, which is ready by then.
  //
  // A reduction with the scan's own combine and init (the same code) over
  // the same tensor is the scan's last element of each row, in the
  // interpreter as in every scan template: it takes those values
  // (same_fold=0 keeps it its own kernels). The reverse-mode adjoint of a
  // row scan, total - prefix + adjoint, is such a pair: computed from one
  // fold, its total and prefixes round together, as the interpreter's do.
  void find_sibling_groups() {
    std::map<int, size_t> pos;
    for (size_t i = 0; i < plan.roots.size(); i++) pos[plan.roots[i]] = i;
    std::set<int> folded_in_map;
    for (auto &fr : fused_red_of_map) folded_in_map.insert(fr.second);
    if (tune("same_fold", 1))
      for (int s : plan.roots) {
        const TNode &sn = g.ts[s];
        if (sn.kind != TK::Scan || sn.numel == 0) continue;
        const int64_t rows = sn.numel / row_length(sn.shape);
        const std::string sc = gen.combine_fn("c_", sn.body, sn.dt), si = gen.const_fn("z_", sn.init, sn.dt);
        for (int r : plan.roots) {
          const TNode &rn = g.ts[r];
          if (rn.kind != TK::Reduce || rn.a != sn.a || rn.dt != sn.dt || rn.numel != rows) continue;
          if (same_fold_red.count(r) || folded_in_map.count(r)) continue;
          if (gen.combine_fn("c_", rn.body, rn.dt) != sc || gen.const_fn("z_", rn.init, rn.dt) != si) continue;
          same_fold_of[s] = r;
          same_fold_red.insert(r);
          break;
        }
      }
    for (int s : plan.roots) {
      const TNode &sn = g.ts[s];
      if (sn.kind != TK::Scan) continue;
      std::vector<int> reds;
      if (tune("sibling_fuse", 1) && scan_is_row_tile(s)) {
        const int64_t len = row_length(sn.shape), rows = sn.numel / len;
        for (int r : plan.roots) {
          const TNode &rn = g.ts[r];
          if (rn.kind != TK::Reduce || rn.a != sn.a || sib_member.count(r) || sib_lead.count(r) ||
              folded_in_map.count(r) || same_fold_red.count(r))
            continue;
          if (row_length(g.ts[rn.a].shape) != len || rn.numel != rows || !reduce_is_tree(r)) continue;
          reds.push_back(r);
        }
      }
      std::vector<int> members = reds;
      const auto sf = same_fold_of.find(s);
      if (sf != same_fold_of.end()) {
        members.push_back(sf->second);
        gen.rowlast_[s] = {buf_of[sf->second], row_length(sn.shape)};
      }
      if (members.empty()) continue;
      int lead = s;
      for (int r : members)
        if (pos[r] < pos[lead]) lead = r;
      sib_reds[s] = reds;
      sib_lead[lead] = s;
      if (lead != s) sib_member.insert(s);
      for (int r : members)
        if (r != lead) sib_member.insert(r);
    }
  }

  // Gathers of the last element of every row of a row scan that folds one
  // lane a row (the Monte Carlo paths' final prices: index p * 64 + 63).
  // The scan also stores each row's fold, which is that element, in a side
  // buffer of one value a row, and the gather reads it there: one
  // contiguous read instead of one cache line per row of the scan's output
  // (rowlast=0 keeps the strided reads). Eligible where the gather's
  // source reaches the scan through element-wise nodes only, so that the
  // scan's buffer is read at the gather's index.
  void find_rowlast_gathers() {
    if (!tune("rowlast", 1)) return;
    std::function<bool(int, int)> reaches = [&](int t, int s) {
      if (t == s) return true;
      if (plan.materialized[t]) return false;
      const TNode &n = g.ts[t];
      switch (n.kind) {
        case TK::Map:
        case TK::Reshape: return reaches(n.a, s);
        case TK::Map2: return reaches(n.a, s) || reaches(n.b, s);
        default: return false;
      }
    };
    for (size_t gi = 0; gi < g.ts.size(); gi++) {
      const TNode &gn = g.ts[gi];
      if (gn.kind != TK::Gather) continue;
      const Aff a = aff_t(gn.a);
      if (!a.ok) continue;
      for (int s : plan.roots) {
        const TNode &sn = g.ts[s];
        const bool map = (sn.kind == TK::Map || sn.kind == TK::Map2) && !gen.uniform(s);
        if ((sn.kind != TK::Scan && !map) || !plan.materialized[s] || sn.numel == 0) continue;
        const int64_t L = row_length(sn.shape), R = sn.numel / L;
        if (L < 2 || a.a != L || a.b != L - 1 || gn.numel != R) continue;
        // a scan: the template that folds one lane a row, as lower_scan
        // chooses it; a map root: the map template, which stores each
        // row's last element as it computes it
        if (!map && !(R >= 1024 && !(tune("rs_tree", 1) && L >= tune("rs_tree_len", 2048) &&
                                     any_order(sn.body, sn.dt, true))))
          continue;
        if (!reaches(gn.b, s)) continue;
        if (!gen.rowlast_.count(s))
          gen.rowlast_[s] = {add_buf("t" + std::to_string(sn.id) + "_last", sn.dt, R, BufRole::Computed), L};
        gen.rowlast_gather_[(int)gi] = s;
        break;
      }
    }
  }

  std::vector<int> lower_scan(int t, const std::vector<int> &reds = {}) {
    const TNode &n = g.ts[t];
    std::string id = std::to_string(n.id);
    std::string kname = "k_" + id;
    std::string T = dt_ctype(n.dt);
    int out = buf_of[t];
    int64_t len = row_length(n.shape);
    int64_t rows = len == 0 ? 0 : n.numel / len;
    std::string cmb = "c_" + id, ini = "z_" + id;
    src << gen.combine_fn(cmb, n.body, n.dt) << gen.const_fn(ini, n.init, n.dt);
    // sibling reductions folded in this kernel: their combines, inits, types
    std::vector<std::string> rcmb, rini, rT;
    std::vector<int> rout;
    for (int r : reds) {
      const TNode &rn = g.ts[r];
      const std::string rid = std::to_string(rn.id);
      rcmb.push_back("c_" + rid);
      rini.push_back("z_" + rid);
      rT.push_back(dt_ctype(rn.dt));
      rout.push_back(buf_of[r]);
      src << gen.combine_fn(rcmb.back(), rn.body, rn.dt) << gen.const_fn(rini.back(), rn.init, rn.dt);
    }
    if (rows == 0) return {};
    ElemFn f = gen.element_fn("f_" + id, n.a, false, true);
    src << f.code;
    // a side buffer of each row's last element (Gen::rowlast_): the tile
    // and wave templates store it here, the row-sequential one on its own
    const auto sd = gen.rowlast_.find(t);
    const int side = sd != gen.rowlast_.end() ? sd->second.first : -1;
    // 1024 rows or more scan one lane a row, in order, unless the rows are
    // long (rs_tree_len) and the combine allows any grouping (bit-exact for
    // max, min and integer ops; float add and mul within rounding): those
    // take the tile templates below, a workgroup a row, or a look-back
    // chain of tiles where a row is longer than one tile. 2^28 f32 or i32
    // elements, µs in order against as tiles: 8192 long 475-480 / 375-381,
    // 4096 long 427-429 / 340-344, 2048 long 411-430 / 363-373, 1000 long
    // 501-504 / 538-569, 256 long 401-405 / 1453-1572. rs_tree=0 scans
    // every row in order (bit-identical to the interpreter).
    if (rows >= 1024 &&
        !(tune("rs_tree", 1) && len >= tune("rs_tree_len", 2048) && any_order(n.body, n.dt, true)))
      return lower_rows_seq(t, true, f, cmb, ini, rows, len);
    bool wide = dt_size(n.dt) == 8;
    if (len <= 64) {
      int64_t S = pow2ceil(len);
      int64_t rpw = 64 / S;
      Params p;
      add_in(p, f);
      p.out.push_back(out);
      if (side >= 0) p.out.push_back(side);
      std::vector<int> args;
      std::string params = param_list(p, args);
      std::ostringstream k;
      k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "(" << params << ") {\n"
        << "  const int lane = threadIdx.x & 63;\n"
        << "  const int seg = lane / " << S << ";\n"
        << "  const int sl = lane - seg * " << S << ";\n"
        << "  const int wave = (blockIdx.x * 256 + threadIdx.x) >> 6;\n"
        << "  const int nwaves = gridDim.x * 4;\n"
        << "  for (int rb = wave * " << rpw << "; rb < " << rows << "; rb += nwaves * " << rpw << ") {\n"
        << "    const int r = rb + seg;\n"
        << "    const bool valid = r < " << rows << " && sl < " << len << ";\n"
        << "    const int i = r * " << len << " + sl;\n"
        << "    " << T << " v = " << ini << "();\n"
        << "    if (valid) v = " << f.call_scalar("i") << ";\n"
        << "    if (sl == 0) v = " << cmb << "(" << ini << "(), v);\n";
      for (int64_t off = 1; off < S; off *= 2)
        k << "    { const " << T << " u = __shfl_up(v, " << off << "); if (sl >= " << off << ") v = " << cmb
          << "(u, v); }\n";
      k << "    if (valid) b" << out << "[i] = v;\n";
      if (side >= 0) k << "    if (valid && sl == " << len - 1 << ") b" << side << "[r] = v;\n";
      k << "  }\n}\n";
      src << k.str();
      int64_t waves = cdiv(rows, rpw);
      int grid = (int)std::min<int64_t>(cdiv(waves, 4), 65536);
      return {add_kernel(kname, args, grid, 256, "scan_wave")};
    }
    // Rows longer than 64 with few rows: a register-resident tile scan.
    // A tile is U slices of 1024 elements; thread t holds the 4 contiguous
    // elements 4t..4t+3 of every slice (one 16-byte load each, all in
    // flight together). The scan runs in that layout: a 4-element scan per
    // thread, a wave scan of thread totals per slice, one barrier to share
    // the 4 wave totals of every slice, and the slice prefixes are folded
    // in with earlier elements always on the left. When a row spans
    // several tiles they are chained by a single-pass decoupled look-back;
    // status words carry the flag (1 aggregate, 2 inclusive prefix) in the
    // high half and the value bits in the low half (8-byte values use two
    // words, each tagged).
    //
    // Which tile a workgroup takes: for 4-byte values, its own blockIdx.
    // Nothing then makes a predecessor's workgroup run before its
    // successors, so the look-back never waits unboundedly: after lb_spin
    // polls of a predecessor that has published nothing, the waiting wave
    // reads that tile's elements and folds them itself (tile_fold: each
    // lane a contiguous share, then the lanes in a tree, earlier elements
    // always on the left) and goes on. Progress is guaranteed whatever the
    // dispatch order; with the usual in-order dispatch the fallback is
    // never taken. That grouping is not the tile's own (4 elements per
    // thread, a wave scan, then wave and slice totals), so for float add
    // the fallback rounds differently: a float look-back scan is not
    // bit-reproducible from run to run when the fallback fires. Integer,
    // min and max scans are exact in any grouping.
    // 8-byte values take tiles in launch order from an atomic counter, so
    // a tile only waits on tiles whose workgroups are already running.
    // Waves per workgroup (4 or 8); a slice is 4 elements per thread. 8
    // waves stream fastest on gfx950. 4-byte values over 13 slices (26624
    // elements a tile): 2^28 i32 in 381-383 us, against 395-398 us for 4
    // waves over 22 slices, and 386, 396, 392 and 397 us for 8 waves over
    // 12, 14, 15 and 16 slices. 8-byte values over 8 slices: 2^27 i64 or
    // f64 in 472-476 us, against 552 us for 4 waves (6 slices: the same;
    // 4, 5 and 7 slices: 545, 493-519 and 485 us).
    const TileShape ts = tile_shape(len, n.dt);
    const int64_t NW = ts.NW, SL = ts.SL, NT = 64 * NW, U = ts.U, tile = ts.tile, tpr = ts.tpr;
    int64_t tiles = rows * tpr;
    bool chained = tpr > 1;
    if (!reds.empty() && chained) throw Failure("Lower: sibling reductions need one tile a row");
    bool vec = len % 4 == 0;
    int words = wide ? 2 : 1;
    const bool selfsched = chained && !wide && tune("lb_counter", 0) == 0;
    int status = -1, ctr = -1, kinit = -1;
    if (chained) {
      status = add_buf("t" + id + "_status", DT::I64, tiles * words, BufRole::Scratch);
      if (!selfsched) ctr = add_buf("t" + id + "_tiles", DT::I32, 2, BufRole::Scratch);
      need_err = true;
      std::string iname = kname + "_init";
      std::ostringstream k;
      k << "extern \"C\" __global__ __launch_bounds__(256) void " << iname << "(long long* __restrict__ b" << status;
      if (!selfsched) k << ", int* __restrict__ b" << ctr;
      k << ") {\n"
        << "  const int stride = gridDim.x * 256;\n"
        << "  for (int q = blockIdx.x * 256 + threadIdx.x; q < " << tiles * words << "; q += stride) b" << status
        << "[q] = 0;\n";
      if (!selfsched) k << "  if (blockIdx.x == 0 && threadIdx.x < 2) b" << ctr << "[threadIdx.x] = 0;\n";
      k << "}\n";
      src << k.str();
      std::vector<int> iargs = {status};
      if (!selfsched) iargs.push_back(ctr);
      kinit = add_kernel(iname, iargs, (int)std::min<int64_t>(cdiv(tiles * words, 256), 1024), 256, "scan_init");
    }
    Params p;
    add_in(p, f);
    p.out.push_back(out);
    for (int o : rout) p.out.push_back(o);
    if (side >= 0) p.out.push_back(side);
    if (chained) p.err = true;
    std::vector<int> args;
    std::string params = param_list(p, args);
    if (chained) {
      args.push_back(status);
      if (!selfsched) args.push_back(ctr);
    }
    std::string pub;
    if (!wide) {
      pub =
          "__hip_atomic_store(&st[TILE], ((cc_u64)(FLAG) << 32) | cc_bits(VAL), __ATOMIC_RELAXED, "
          "__HIP_MEMORY_SCOPE_AGENT)";
    } else {
      pub =
          "{ const cc_u64 bb = cc_bits(VAL); "
          "__hip_atomic_store(&st[2 * (TILE)], ((cc_u64)(FLAG) << 32) | (bb & 0xffffffffull), __ATOMIC_RELAXED, "
          "__HIP_MEMORY_SCOPE_AGENT); "
          "__hip_atomic_store(&st[2 * (TILE) + 1], ((cc_u64)(FLAG) << 32) | (bb >> 32), __ATOMIC_RELAXED, "
          "__HIP_MEMORY_SCOPE_AGENT); }";
    }
    auto publish = [&](const std::string &tl, const std::string &flag, const std::string &val) {
      std::string r = pub;
      auto rep = [&](const std::string &a, const std::string &b) {
        size_t q = 0;
        while ((q = r.find(a, q)) != std::string::npos) {
          r.replace(q, a.size(), b);
          q += b.size();
        }
      };
      rep("TILE", tl);
      rep("FLAG", flag);
      rep("VAL", val);
      return r;
    };
    // Buffer-resource loads and stores (one shared offset register for the
    // whole tile): 4-byte operands under 2 GiB, and an element function
    // without gathers, since lanes past the tile read (and discard) data
    // beyond it.
    bool bufx = vec && tune("lb_buf", 1) && f.ptrs.empty() && dt_size(n.dt) == 4 &&
                prog.bufs[out].bytes() < (int64_t(1) << 31);
    for (int b : f.ident) bufx = bufx && dt_size(prog.bufs[b].dt) == 4 && prog.bufs[b].bytes() < (int64_t(1) << 31);
    // Streaming (non-temporal) accesses, a bit mask: 1 stores, 2 loads.
    // Look-back scans stream both; one-tile-a-row scans stream their stores
    // only (config 2's step 0.482-0.484 -> 0.475-0.477 ms, the rows kernel
    // 96 -> 89 us: their plain loads leave clean lines in the MALL where
    // streamed ones measured slower; rt_nt=3 streams both).
    int64_t scan_nt = tune(chained ? "scan_nt" : "rt_nt", -1);
    if (scan_nt < 0)
      scan_nt = narrow(f, n.dt) && streams(fn_bytes(f, rows * len) + rows * len * dt_size(n.dt)) ? (chained ? 3 : 1) : 0;
    if (n.dt == DT::BOOL) scan_nt = 0;
    for (int b : f.ident)
      if (prog.bufs[b].dt == DT::BOOL) scan_nt &= ~int64_t(2);
    static const char *comp[] = {"x", "y", "z", "w"};
    std::ostringstream k;
    // Four waves per SIMD (at most 128 VGPRs): the fallback's registers
    // must not cost the main path its occupancy.
    k << "extern \"C\" __global__ __launch_bounds__(" << NT << ") "
      << (selfsched ? "__attribute__((amdgpu_waves_per_eu(4))) " : "") << "void " << kname << "(" << params;
    if (chained) k << ", cc_u64* __restrict__ st" << (selfsched ? "" : ", int* __restrict__ ctr");
    k << ") {\n"
      << "  __shared__ " << T << " wsum[" << U << "][" << NW << "];\n"
      << "  __shared__ " << T << " s_prefix;\n"
      << "  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;\n";
    for (size_t j = 0; j < reds.size(); j++)
      k << "  __shared__ " << rT[j] << " rpart" << j << "[" << NW << "];\n"
        << "  __shared__ bool rhas" << j << "[" << NW << "];\n";
    if (chained && !selfsched) {
      k << "  __shared__ int s_tile;\n"
        << "  if (threadIdx.x == 0) s_tile = atomicAdd(ctr, 1);\n"
        << "  __syncthreads();\n"
        << "  const int tile = s_tile;\n";
    } else {
      k << "  const int tile = blockIdx.x;\n";
    }
    k << "  const int row = tile / " << tpr << ";\n"
      << "  const int tin = tile - row * " << tpr << ";\n"
      << "  const int base = row * " << len << " + tin * " << tile << ";\n"
      << "  const int tl = min(" << tile << ", " << len << " - tin * " << tile << ");\n";
    if (bufx) {
      for (int b : f.ident)
        k << "  const __amdgpu_buffer_rsrc_t r" << b << " = cc_rsrc(b" << b << ", " << prog.bufs[b].bytes() << "u);\n";
      k << "  const __amdgpu_buffer_rsrc_t ro = cc_rsrc(b" << out << ", " << prog.bufs[out].bytes() << "u);\n";
    }
    k << "  " << T << " v[" << U << "][4];\n"
      << "#pragma unroll\n"
      << "  for (int u = 0; u < " << U << "; u++) {\n"
      << "    const int e = threadIdx.x * 4 + " << SL << " * u;\n";
    // Groups past the tile read the tile's first group (always valid) and
    // take init: no load sits behind a branch.
    if (vec) {
      k << "    const bool ok = e < tl;\n"
        << "    const int i = base + (ok ? e : 0);\n";
      if (bufx) {
        for (int b : f.ident)
          k << "    const cc_v4<" << ty(b) << "> l" << b << " = cc_bld4<" << ty(b) << ", " << ((scan_nt & 2) ? 2 : 0)
            << ">(r" << b << ", threadIdx.x * 16, (base + " << SL << " * u) * 4);\n";
      } else {
        k << vec_loads(f, "i", "    ", tyof(), (scan_nt & 2) != 0);
      }
      for (int c = 0; c < 4; c++)
        k << "    v[u][" << c << "] = ok ? " << lane_call(f, "i", c) << " : " << ini << "();\n";
    } else {
      for (int c = 0; c < 4; c++)
        k << "    { const bool ok = e + " << c << " < tl; const int i = base + (ok ? e + " << c << " : 0); v[u][" << c
          << "] = ok ? " << f.call_scalar("i") << " : " << ini << "(); }\n";
    }
    k << "  }\n";
    // Sibling reductions: each lane folds its elements in row order (slice
    // by slice) before the scan changes them, then the wave in a butterfly;
    // one partial a wave goes to LDS with the scan's wave totals.
    for (size_t j = 0; j < reds.size(); j++) {
      const std::string A = "racc" + std::to_string(j), Hs = "rh" + std::to_string(j);
      k << "  " << rT[j] << " " << A << " = " << rini[j] << "();\n"
        << "  bool " << Hs << " = false;\n"
        << "#pragma unroll\n"
        << "  for (int u = 0; u < " << U << "; u++) {\n"
        << "    const int e = threadIdx.x * 4 + " << SL << " * u;\n"
        << "#pragma unroll\n"
        << "    for (int c = 0; c < 4; c++) {\n"
        << "      const bool ok_ = e + c < tl;\n"
        << "      const " << rT[j] << " y_ = " << Hs << " ? " << rcmb[j] << "(" << A << ", v[u][c]) : v[u][c];\n"
        << "      " << A << " = ok_ ? y_ : " << A << "; " << Hs << " = " << Hs << " || ok_;\n"
        << "    }\n"
        << "  }\n"
        << "  for (int off = 32; off > 0; off >>= 1) { const " << rT[j] << " o_ = __shfl_xor(" << A
        << ", off); const bool oh_ = __shfl_xor((int)" << Hs << ", off) != 0; if (oh_) { " << A << " = " << Hs
        << " ? " << rcmb[j] << "(" << A << ", o_) : o_; " << Hs << " = true; } }\n"
        << "  if (lane == 0) { rpart" << j << "[wid] = " << A << "; rhas" << j << "[wid] = " << Hs << "; }\n";
    }
    k << "  if (tin == 0 && threadIdx.x == 0) v[0][0] = " << cmb << "(" << ini << "(), v[0][0]);\n"
      << "#pragma unroll\n"
      << "  for (int u = 0; u < " << U << "; u++) {\n"
      << "    v[u][1] = " << cmb << "(v[u][0], v[u][1]);\n"
      << "    v[u][2] = " << cmb << "(v[u][1], v[u][2]);\n"
      << "    v[u][3] = " << cmb << "(v[u][2], v[u][3]);\n"
      << "    " << T << " incl = v[u][3];\n";
    for (int off = 1; off < 64; off *= 2)
      k << "    { const " << T << " o = __shfl_up(incl, " << off << "); if (lane >= " << off << ") incl = " << cmb
        << "(o, incl); }\n";
    // the wave's exclusive prefix is folded in at once (no register per slice kept for it)
    k << "    { const " << T << " ex = __shfl_up(incl, 1);\n"
      << "      if (lane > 0) { v[u][0] = " << cmb << "(ex, v[u][0]); v[u][1] = " << cmb << "(ex, v[u][1]);\n"
      << "                      v[u][2] = " << cmb << "(ex, v[u][2]); v[u][3] = " << cmb << "(ex, v[u][3]); } }\n"
      << "    if (lane == 63) wsum[u][wid] = incl;\n"
      << "  }\n"
      << "  __syncthreads();\n"
      << "  " << T << " run = " << ini << "();\n"
      << "#pragma unroll\n"
      << "  for (int u = 0; u < " << U << "; u++) {\n"
      << "    bool hp = u > 0;\n"
      << "    " << T << " pf = run;\n"
      << "    for (int w = 0; w < wid; w++) { pf = hp ? " << cmb << "(pf, wsum[u][w]) : wsum[u][w]; hp = true; }\n"
      << "    if (hp) {\n"
      << "      v[u][0] = " << cmb << "(pf, v[u][0]); v[u][1] = " << cmb << "(pf, v[u][1]);\n"
      << "      v[u][2] = " << cmb << "(pf, v[u][2]); v[u][3] = " << cmb << "(pf, v[u][3]);\n"
      << "    }\n"
      << "    " << T << " su = wsum[u][0];\n"
      << "#pragma unroll\n"
      << "    for (int w = 1; w < " << NW << "; w++) su = " << cmb << "(su, wsum[u][w]);\n"
      << "    run = u > 0 ? " << cmb << "(run, su) : su;\n"
      << "  }\n";
    // the sibling reductions' wave partials, in wave order (the barrier
    // above made them visible); init once, to the row's total
    for (size_t j = 0; j < reds.size(); j++)
      k << "  if (threadIdx.x == 0) {\n"
        << "    " << rT[j] << " t = " << rini[j] << "();\n"
        << "    bool th = false;\n"
        << "    for (int w = 0; w < " << NW << "; w++) if (rhas" << j << "[w]) { t = th ? " << rcmb[j] << "(t, rpart"
        << j << "[w]) : rpart" << j << "[w]; th = true; }\n"
        << "    b" << rout[j] << "[row] = th ? " << rcmb[j] << "(" << rini[j] << "(), t) : " << rini[j] << "();\n"
        << "  }\n";
    if (chained) {
      k << "  if (threadIdx.x == 0) " << publish("tile", "tin == 0 ? 2 : 1", "run") << ";\n"
        << "  if (tin > 0) {\n"
        << "    if (wid == 0) {\n"
        << "      const int rowstart = row * " << tpr << ";\n"
        << "      " << T << " acc = " << ini << "();\n"
        << "      bool have = false;\n"
        << "      int j = tile - 1;\n"
        << "      unsigned spins = 0;\n"
        << "      while (true) {\n";
      if (!wide) {
        // K predecessors per lane (lane l covers tiles j - K*l - k, k = 0..K-1,
        // position K*l + k counted from the nearest), all loaded in one round
        // trip. Only words nearer than the nearest inclusive prefix found so
        // far are waited for. K = 1 measures best on gfx950 (2^28 i32: 475 us
        // at K = 1, 503 at 2, 601 at 4): the wait is dominated by
        // predecessors still loading, and more uncached status loads per
        // round only add latency under load.
        const int64_t K = std::max<int64_t>(1, std::min<int64_t>(8, tune("lb_window", 1)));
        std::string sK = std::to_string(K);
        k << "        const int q0 = j - " << sK << " * lane;\n"
          << "        int fl[" << sK << "];\n"
          << "        " << T << " val[" << sK << "];\n"
          << "#pragma unroll\n"
          << "        for (int c = 0; c < " << sK << "; c++) {\n"
          << "          fl[c] = 2; val[c] = " << ini << "();\n"
          << "          if (q0 - c >= rowstart) {\n"
          << "            const cc_u64 w = __hip_atomic_load(&st[q0 - c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);\n"
          << "            fl[c] = (int)(w >> 32); val[c] = cc_from_bits<" << T << ">(w & 0xffffffffull);\n"
          << "          }\n"
          << "        }\n"
          << "        int P;\n"
          << (selfsched ? "        for (;;) {\n        bool timedout = false;\n" : "")
          << "        while (true) {\n"
          << "          int mine = " << sK << ";\n"
          << "#pragma unroll\n"
          << "          for (int c = " << K - 1 << "; c >= 0; c--) if (fl[c] == 2) mine = c;\n"
          << "          const cc_u64 im = __ballot(mine < " << sK << ");\n"
          << "          P = " << 64 * K << ";\n"
          << "          if (im) { const int Lf = __ffsll((long long)im) - 1; P = " << sK
          << " * Lf + __shfl(mine, Lf); }\n"
          << "          bool wait = false;\n"
          << "#pragma unroll\n"
          << "          for (int c = 0; c < " << sK << "; c++) wait |= fl[c] == 0 && " << sK << " * lane + c < P;\n"
          << "          if (!__ballot(wait)) break;\n";
        if (selfsched) {
          // The nearest word still unpublished: its tile is folded here.
          const int64_t spin = std::max<int64_t>(1, tune("lb_spin", 1 << 14));
          k << "          if (++spins > " << spin << "u) { timedout = true; break; }\n";
        } else {
          k << "          if (++spins > (1u << 24)) { cc_flag(err, 4); P = 0;\n"
            << "#pragma unroll\n"
            << "            for (int c = 0; c < " << sK << "; c++) { fl[c] = 2; val[c] = " << ini << "(); }\n"
            << "            break; }\n";
        }
        k << "          __builtin_amdgcn_s_sleep(1);\n"
          << "#pragma unroll\n"
          << "          for (int c = 0; c < " << sK << "; c++)\n"
          << "            if (fl[c] == 0 && " << sK << " * lane + c < P) {\n"
          << "              const cc_u64 w = __hip_atomic_load(&st[q0 - c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);\n"
          << "              fl[c] = (int)(w >> 32); val[c] = cc_from_bits<" << T << ">(w & 0xffffffffull);\n"
          << "            }\n"
          << "        }\n";
        if (selfsched) {
          // Out of the polling loop on the spin limit: the nearest word still
          // unpublished has its tile folded here, then polling resumes.
          const int64_t spin = std::max<int64_t>(1, tune("lb_spin", 1 << 14));
          // Taken only when the polling loop stopped on the limit, which it
          // checks after finding a word still awaited: some lane then has
          // one (mz < K), so Lz is a lane.
          k << "        if (!timedout) break;\n"
            << "        {\n"
            << "            int mz = " << sK << ";\n"
            << "#pragma unroll\n"
            << "            for (int c = " << K - 1 << "; c >= 0; c--) if (fl[c] == 0 && " << sK << " * lane + c < P) mz = c;\n"
            << "            const int Lz = __ffsll((long long)__ballot(mz < " << sK << ")) - 1;\n"
            << "            const int cz = __shfl(mz, Lz);\n"
            << "            const int q = j - (" << sK << " * Lz + cz);\n"
            << tile_fold(f, cmb, ini, T, U, tpr, len, tile)
            << "#pragma unroll\n"
            << "            for (int c = 0; c < " << sK << "; c++)\n"
            << "              if (lane == Lz && c == cz) { fl[c] = tq == 0 ? 2 : 1; val[c] = agg; }\n"
            << "            spins = " << std::max<int64_t>(0, spin - 8) << "u;\n"
            << "        }\n"
            << "        }\n";
        }
        k
          // lane-local fold, farthest word first, of the positions <= P
          << "        " << T << " w = " << ini << "();\n"
          << "        bool hw = false;\n"
          << "#pragma unroll\n"
          << "        for (int c = " << K - 1 << "; c >= 0; c--)\n"
          << "          if (" << sK << " * lane + c <= P) { w = hw ? " << cmb << "(w, val[c]) : val[c]; hw = true; }\n";
        k << lookback_tree(cmb, T)
          << "        w = __shfl(w, 0);\n"
          << "        acc = have ? " << cmb << "(w, acc) : w;\n"
          << "        have = true;\n"
          << "        if (P < " << 64 * K << ") break;\n"
          << "        j -= " << 64 * K << ";\n"
          << "      }\n";
      } else {
        k << "        const int q = j - lane;\n"
          << "        int flag = 2;\n"
          << "        " << T << " val = " << ini << "();\n"
          << "        if (q >= rowstart) {\n"
          << "          while (true) {\n"
          << "            const cc_u64 w0 = __hip_atomic_load(&st[2 * q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);\n"
          << "            const cc_u64 w1 = __hip_atomic_load(&st[2 * q + 1], __ATOMIC_RELAXED, "
             "__HIP_MEMORY_SCOPE_AGENT);\n"
          << "            flag = (int)(w0 >> 32);\n"
          << "            if (flag != 0 && flag == (int)(w1 >> 32)) { val = cc_from_bits<" << T
          << ">((w0 & 0xffffffffull) | (w1 << 32)); break; }\n"
          << "            if (++spins > (1u << 24)) { cc_flag(err, 4); flag = 2; break; }\n"
          << "            __builtin_amdgcn_s_sleep(1);\n"
          << "          }\n"
          << "        }\n"
          << "        const cc_u64 pm = __ballot(flag == 2);\n"
          << "        const int L = pm ? (__ffsll((long long)pm) - 1) : 63;\n"
          << "        " << T << " w = val;\n"
          << "        bool hw = lane <= L;\n";
        k << lookback_tree(cmb, T)
          << "        w = __shfl(w, 0);\n"
          << "        acc = have ? " << cmb << "(w, acc) : w;\n"
          << "        have = true;\n"
          << "        if (pm) break;\n"
          << "        j -= 64;\n"
          << "      }\n";
      }
      k
        << "      if (lane == 0) {\n"
        << "        s_prefix = acc;\n"
        << "        const " << T << " incl = " << cmb << "(acc, run);\n"
        << "        " << publish("tile", "2", "incl") << ";\n"
        << "      }\n"
        << "    }\n"
        << "    __syncthreads();\n"
        << "    const " << T << " pfx = s_prefix;\n"
        << "#pragma unroll\n"
        << "    for (int u = 0; u < " << U << "; u++) {\n"
        << "      v[u][0] = " << cmb << "(pfx, v[u][0]); v[u][1] = " << cmb << "(pfx, v[u][1]);\n"
        << "      v[u][2] = " << cmb << "(pfx, v[u][2]); v[u][3] = " << cmb << "(pfx, v[u][3]);\n"
        << "    }\n"
        << "  }\n";
    }
    k << "#pragma unroll\n"
      << "  for (int u = 0; u < " << U << "; u++) {\n"
      << "    const int e = threadIdx.x * 4 + " << SL << " * u;\n";
    if (vec) {
      k << "    if (e < tl) {\n"
        << "      cc_v4<" << T << "> o;\n";
      for (int c = 0; c < 4; c++) k << "      o." << comp[c] << " = v[u][" << c << "];\n";
      if (bufx)
        k << "      cc_bst4<" << T << ", " << ((scan_nt & 1) ? 2 : 0)
          << ">(ro, threadIdx.x * 16, (base + " << SL << " * u) * 4, o);\n";
      else if (scan_nt & 1)
        k << "      cc_st4_nt(b" << out << " + base + e, o);\n";
      else
        k << "      *(cc_v4<" << T << ">*)(b" << out << " + base + e) = o;\n";
      k << "    }\n";
    } else {
      for (int c = 0; c < 4; c++)
        k << "    if (e + " << c << " < tl) b" << out << "[base + e + " << c << "] = v[u][" << c << "];\n";
    }
    // the row's last element, held by one thread of the row's last tile
    if (side >= 0)
      k << "    if (tin == " << tpr - 1 << ")\n"
        << "#pragma unroll\n"
        << "      for (int c = 0; c < 4; c++) if (e + c == tl - 1) b" << side << "[row] = v[u][c];\n";
    k << "  }\n"
      << "}\n";
    src << k.str();
    int kscan = add_kernel(kname, args, (int)tiles, (int)NT,
                           chained ? "scan_lookback" : reds.empty() ? "scan_tile" : "scan_tile_fold");
    if (chained) return {kinit, kscan};
    return {kscan};
  }

  // ---- Scatter_add without global atomics -----------------------------------
  // Device-wide atomics run at roughly one per clock per XCD whatever the
  // table size, so collisions are resolved in LDS instead. The bins are cut
  // into P slices of S bins (S a power of two, S * sizeof(T) <= 64 KiB):
  //   count     chunk g counts its elements per slice      -> cnt[g][p]
  //   colscan   cnt[g][p] becomes the offset of chunk g within slice p,
  //             start[p] the slice's total
  //   bscan     start[] becomes the exclusive prefix of the totals
  //   partition chunk g writes (bin within slice, value) pairs into slice
  //             order at start[p] + cnt[g][p] + (rank within the chunk)
  //   accumulate W workgroups per slice fold the slice's pairs into an LDS
  //             table with LDS atomics and store it (W = 1) or a partial
  //   reduce    out[b] = sum over w of the partials, w ascending
  // With one slice (B <= S) the partition is skipped and the workgroups
  // fold contiguous input chunks directly. Out-of-range indices are skipped
  // and flag error 2, as the atomic path does. Within a slice the order of
  // the additions depends on LDS arrival order, so float sums are not
  // bit-reproducible (the atomic path's are not either).
  // The largest power of two below n (1 for n <= 2): the first step of a
  // binary search over n sorted entries.
  static int64_t top_pow2(int64_t n) {
    int64_t t = 1;
    while (t * 2 < n) t *= 2;
    return t;
  }
  // Emitted code: the windows of super-slice `Q` of a windowed pass are
  // tiles [ta_, tz_).
  static std::string windows_of(const PassOut &o, const std::string &Q) {
    std::ostringstream l;
    l << "  const int ta_ = b" << o.wtab << "[" << Q << "], tz_ = b" << o.wtab << "[" << Q << " + 1];\n";
    return l.str();
  }
  // Emitted code: window `ft` of a windowed pass: its super-slice Q_ (the
  // last whose first window is at or before ft, found in LDS), its first
  // element wb_ and length wn_ in the coarse output. Has a barrier; the
  // whole workgroup returns for a window past the last one.
  static std::string window_at(const PassOut &o, const std::string &ft) {
    std::ostringstream l;
    l << "  __shared__ int wt_[" << o.P1 + 1 << "];\n"
      << "  if (threadIdx.x <= " << o.P1 << ") wt_[threadIdx.x] = b" << o.wtab << "[threadIdx.x];\n"
      << "  __syncthreads();\n"
      << "  if (" << ft << " >= wt_[" << o.P1 << "]) return;\n"
      << "  int Q_ = 0;\n"
      << "#pragma unroll\n"
      << "  for (int st = " << top_pow2(o.P1) << "; st >= 1; st >>= 1)\n"
      << "    if (Q_ + st < " << o.P1 << " && wt_[Q_ + st] <= " << ft << ") Q_ += st;\n"
      << "  const int* const s1_ = b" << o.wstart << ";\n"
      << "  const int wb_ = s1_[Q_] + (" << ft << " - wt_[Q_]) * " << o.TILE << ";\n"
      << "  const int wn_ = s1_[Q_ + 1] - wb_ < " << o.TILE << " ? s1_[Q_ + 1] - wb_ : " << o.TILE << ";\n";
    return l.str();
  }

  // The runs of slice q over tiles [t_lo, t_hi) of a tile-local partition
  // (`o`), 8 elements a lane, `ug` groups of 8 a lane in flight (UG_). Each wave
  // takes `tpw` tiles at a time (64, or fewer where a workgroup is expected
  // to have few tiles, so that every wave gets some): their run lengths in
  // groups of 8 are summed across the wave, and a lane finds its group's
  // tile by a binary search over those sums, so that consecutive lanes read
  // consecutive groups. `loads` then `body` are emitted with pos_[u] (the
  // group's first element) and nv_[u] (its valid elements; 0 for a lane
  // without a group, whose pos_ still points into the pair arrays) for
  // u in [0, UG_) in scope.
  static std::string runs_walk(const PassOut &o, int64_t threads, int64_t tiles_per_wg, const std::string &loads,
                               const std::string &body, int64_t ug = 2) {
    int64_t tpw = 64;
    while (tpw > 1 && tpw * (threads / 64) > tiles_per_wg) tpw /= 2;
    std::ostringstream l;
    l << "  {\n"
      << "    const int2* const runs_ = (const int2*)b" << o.meta << " + (size_t)" << (o.windows ? "(q & 63)" : "q")
      << " * " << o.NTT << ";\n"
      << "    const int lane_ = threadIdx.x & 63;\n"
      << "    for (int tb = t_lo + (int)(threadIdx.x >> 6) * " << tpw << "; tb < t_hi; tb += " << tpw * (threads / 64)
      << ") {\n"
      << "      const int2 m_ = lane_ < " << tpw << " && tb + lane_ < t_hi ? runs_[tb + lane_] : make_int2(0, 0);\n"
      << "      const int ng_ = (m_.y + 7) >> 3;\n"
      << "      int in_ = ng_;\n"
      << "#pragma unroll\n"
      << "      for (int d = 1; d < 64; d <<= 1) {\n"
      << "        const int o_ = __shfl_up(in_, d);\n"
      << "        if (lane_ >= d) in_ += o_;\n"
      << "      }\n"
      << "      const int tot_ = __shfl(in_, 63), ex_ = in_ - ng_;\n"
      << "      constexpr int UG_ = " << ug << ";\n"
      << "      for (int k0 = 0; k0 < tot_; k0 += 64 * UG_) {\n"
      << "        size_t pos_[UG_];\n"
      << "        int nv_[UG_];\n"
      << "#pragma unroll\n"
      << "        for (int u = 0; u < UG_; u++) {\n"
      << "          const int j = k0 + u * 64 + lane_;\n"
      << "          int i = 0;\n"
      << "#pragma unroll\n"
      << "          for (int st = 32; st >= 1; st >>= 1) {\n"
      << "            const int c = __shfl(in_, i + st - 1);\n"
      << "            if (c <= j) i += st;\n"
      << "          }\n"
      << "          const int e0 = __shfl(ex_, i), off = __shfl(m_.x, i), cnt = __shfl(m_.y, i);\n"
      << "          const bool ok = j < tot_;\n"
      << "          pos_[u] = (size_t)(ok ? tb + i : tb) * " << o.RS << " + (ok ? off + 8 * (j - e0) : 0);\n"
      << "          nv_[u] = ok ? min(8, cnt - 8 * (j - e0)) : 0;\n"
      << "        }\n"
      << loads << body << "      }\n"
      << "    }\n"
      << "  }\n";
    return l.str();
  }

  std::vector<int> lower_scatter_lds(int t, int64_t B, int64_t N, int64_t S, int64_t P) {
    const TNode &n = g.ts[t];
    std::string id = std::to_string(n.id);
    std::string kname = "k_" + id;
    std::string T = dt_ctype(n.dt);
    const int64_t ES = dt_size(n.dt);
    int out = buf_of[t];
    int shift = 0;
    while ((int64_t(1) << shift) < S) shift++;
    // inputs read at the element's own index come in by value, so whole
    // 4-element groups can be loaded with 16-byte accesses
    ElemFn fi = gen.element_fn("fi_" + id, n.a, false, true);
    ElemFn fs = gen.element_fn("fs_" + id, n.b, false, true);
    src << fi.code << fs.code;
    std::string acc = n.dt == DT::I32 ? "cc_u32" : T;  // partial sums wrap for i32
    std::vector<int> ks;
    // Loop over [lo, hi) four strides at a time, loads issued first. The
    // clamped index keeps every load in range.
    // Eight strides per iteration: all loads first (clamped to the chunk's
    // first index), then the bodies under an in-range flag rather than a
    // break, so the compiler keeps the loads together.
    auto chunk_loop = [&](bool with_val, const std::string &body) {
      std::ostringstream l;
      l << "  for (int i0 = lo + (int)threadIdx.x; i0 < hi; i0 += 2048) {\n"
        << "    int jj[8];\n";
      if (with_val) l << "    " << T << " xx[8];\n";
      l << "#pragma unroll\n"
        << "    for (int u = 0; u < 8; u++) {\n"
        << "      const int i = i0 + u * 256 < hi ? i0 + u * 256 : lo;\n"
        << "      jj[u] = " << fi.call_scalar("i") << ";\n";
      if (with_val) l << "      xx[u] = " << fs.call_scalar("i") << ";\n";
      l << "    }\n"
        << "#pragma unroll\n"
        << "    for (int u = 0; u < 8; u++) {\n"
        << "      const bool in = i0 + u * 256 < hi;\n"
        << "      const int j = jj[u];\n"
        << body << "    }\n"
        << "  }\n";
      return l.str();
    };
    auto finish = [&](int64_t W, int64_t nslices, int64_t part_bins) {
      // partial tables, then the fixed-order sum
      if (W == 1) return -1;
      int part = add_buf("t" + id + "_part", n.dt, W * part_bins, BufRole::Scratch);
      (void)nslices;
      return part;
    };
    if (P == 1) {
      // One slice: fold input chunks straight into LDS.
      int64_t W = std::min<int64_t>(tune("scatter_direct_wgs", 1024), cdiv(N, 8192));
      W = std::max<int64_t>(1, W);
      int64_t C = cdiv(cdiv(N, W), 256) * 256;
      W = cdiv(N, C);
      int part = finish(W, 1, B);
      Params p;
      add_in(p, fi);
      add_in(p, fs);
      p.out.push_back(part >= 0 ? part : out);
      p.err = true;
      std::vector<int> args;
      std::string params = param_list(p, args);
      int dst = part >= 0 ? part : out;
      std::ostringstream k;
      k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "_direct(" << params << ") {\n"
        << "  __shared__ " << T << " h[" << B << "];\n"
        << "  for (int b = threadIdx.x; b < " << B << "; b += 256) h[b] = " << zero_of(n.dt) << ";\n"
        << "  __syncthreads();\n"
        << "  const int lo = blockIdx.x * " << C << ";\n"
        << "  const int hi = lo + " << C << " < " << N << " ? lo + " << C << " : " << N << ";\n"
        << chunk_loop(true, "      if (in) { if ((unsigned)j < " + std::to_string(B) +
                                "u) cc_lds_add(&h[j], xx[u]); else cc_flag(err, 2); }\n")
        << "  __syncthreads();\n"
        << "  for (int b = threadIdx.x; b < " << B << "; b += 256) b" << dst << "[(size_t)blockIdx.x * " << B
        << " + b] = h[b];\n"
        << "}\n";
      src << k.str();
      ks.push_back(add_kernel(kname + "_direct", args, (int)W, 256, "scatter_direct"));
      if (part >= 0) ks.push_back(scatter_reduce(kname, T, acc, part, out, W, B, B));
      return ks;
    }
    // Workgroups per slice, about 512 in all: for 2^26 values into 2^20
    // bins (64 slices of 16384, 8 each) the accumulate takes 121 us and the
    // fixed-order sum of the partial tables 11 us, against 132 and 17 us
    // with 16 each.
    int64_t W = std::max<int64_t>(1, std::min<int64_t>(16, tune("scatter_slice_wgs", 512) / P));
    while (W > 1 && W * P * S * ES > (int64_t(256) << 20)) W--;
    int part = finish(W, P, P * S);
    std::string sB = std::to_string(B);
    // Partition tile, per pass: 8192 elements where a pass has at most 1024
    // buckets (runs twice as long per bucket as with 4096, at half the
    // occupancy: config 3's partition 323 -> 278 us, config 3b's coarse
    // pass 302 -> 269 us), 4096 above (config 3b's fine pass: 339 against
    // 409 us); scatter_tile forces one size.
    // 1024 threads per staged partition workgroup (config 3's partition
    // 320 -> 288 us, config 3b's passes 313 / 370 -> 282 / 295 us, against
    // 256; 512 is in between); 256 and 512 by scatter_part_threads.
    const int64_t part_threads = tune("scatter_part_threads", 1024) == 256 ? 256
                                 : tune("scatter_part_threads", 1024) == 512 ? 512 : 1024;
    auto tile_of = [&](int64_t PB) -> int64_t {
      const int64_t t = tune("scatter_tile", 0);
      if (t == 4096 || t == 8192) return t;
      return PB <= 1024 ? 8192 : 4096;
    };

    // One partition pass: elements [0, nvalid) of an input stream are
    // grouped by bucket (j >> SH, PB buckets) into key/val arrays in bucket
    // order. `jx`/`xx` give the code for element i's index and value;
    // `check` bounds-checks the index against the bins (first pass only).
    struct PassIn {
      Params p;
      std::function<std::string(const std::string &)> jx, xx;
      // 4-element groups at a multiple of 4: the loads of a group at i (the
      // indices only, or indices and values), then element k's index and
      // value from them
      std::function<std::string(const std::string &)> vload_j, vload_jx;
      std::function<std::string(const std::string &, int)> jv, xv;
      std::string nvalid;
      int nbuf = -1;  // buffer `nvalid` reads, if any
      bool check;
    };
    auto pass = [&](const std::string &sfx, const PassIn &in, int SH, int64_t PB, bool staged, bool final_keys,
                    const std::string &part_role, bool keep, bool local) {
      const int64_t TILE = tile_of(PB);
      // Chunks of at least 4096 elements; 1024 of them for counted passes,
      // and for tile-local runs at least one a tile, so that each
      // workgroup takes one tile and the resident workgroups read one
      // window of the index and value streams (config 3's partition: 229 us
      // over 8 tiles a workgroup, 203 us over one; counted passes measured
      // the same either way).
      const int64_t G_def = local ? std::max<int64_t>(1024, cdiv(N, TILE)) : 1024;
      int64_t G = std::max<int64_t>(1, std::min<int64_t>(tune("scatter_chunks", G_def), cdiv(N, 4096)));
      int64_t C = cdiv(cdiv(N, G), 256) * 256;
      G = cdiv(N, C);
      PassOut o;
      o.G = G;
      o.C = C;
      o.TILE = TILE;
      o.TPC = cdiv(C, TILE);
      o.PB = PB;
      o.nvalid = in.nvalid;
      o.nbuf = in.nbuf;
      o.first = in.check;
      o.local = local;
      if (local) {
        // regions of RS elements: the tile (at most a chunk long) plus at
        // most 7 of padding per bucket, rounded to a multiple of 8
        o.NTT = G * o.TPC;
        o.RS = std::min(TILE, C) + 8 * PB;
        o.key = add_buf("t" + id + "_key" + sfx, DT::I32, cdiv(o.NTT * o.RS, 2), BufRole::Scratch);  // 16-bit keys
        o.val = add_buf("t" + id + "_val" + sfx, n.dt, o.NTT * o.RS, BufRole::Scratch);
        o.meta = add_buf("t" + id + "_runs" + sfx, DT::I32, 2 * (PB + 1) * o.NTT, BufRole::Scratch);
        if (keep) o.slot = add_buf("t" + id + "_slot" + sfx, DT::I32, cdiv(N, 2), BufRole::Scratch);
      } else {
        o.cnt = add_buf("t" + id + "_cnt" + sfx, DT::I32, G * PB, BufRole::Scratch);
        o.start = add_buf("t" + id + "_start" + sfx, DT::I32, PB + 1, BufRole::Scratch);
        o.key = final_keys ? add_buf("t" + id + "_key" + sfx, DT::I32, cdiv(N, 2), BufRole::Scratch)  // 16-bit keys
                           : add_buf("t" + id + "_key" + sfx, DT::I32, N, BufRole::Scratch);
        o.val = add_buf("t" + id + "_val" + sfx, n.dt, N, BufRole::Scratch);
      }
      if (keep && !local) {
        // for a gather back through this partition: each element's slot in
        // its tile's bucket-grouped order (16 bits, 0xffff where the element
        // was skipped), and per tile the bucket runs' starts in the pair
        // arrays and within the tile
        o.slot = add_buf("t" + id + "_slot" + sfx, DT::I32, cdiv(N, 2), BufRole::Scratch);
        o.meta = add_buf("t" + id + "_tiles" + sfx, DT::I32, G * o.TPC * o.meta_stride(), BufRole::Scratch);
      }
      const std::string sh = std::to_string(SH), spb = std::to_string(PB);
      auto bounds = [&](const std::string &v) { return in.check ? "(unsigned)" + v + " < " + sB + "u" : std::string("true"); };
      auto chunk_head = [&]() {
        std::ostringstream l;
        l << "  const int nv_ = " << in.nvalid << ";\n"
          << "  const int lo = blockIdx.x * " << C << ";\n"
          << "  const int hi = lo + " << C << " < nv_ ? lo + " << C << " : nv_;\n";
        return l.str();
      };
      // eight strides per iteration: all loads first (clamped to the chunk's
      // first index), then the bodies under an in-range flag
      auto loop8 = [&](bool with_val, const std::string &body) {
        std::ostringstream l;
        l << "  for (int i0 = lo + (int)threadIdx.x; i0 < hi; i0 += 2048) {\n"
          << "    int jj[8];\n";
        if (with_val) l << "    " << T << " xv[8];\n";
        l << "#pragma unroll\n"
          << "    for (int u = 0; u < 8; u++) {\n"
          << "      const int i = i0 + u * 256 < hi ? i0 + u * 256 : lo;\n"
          << "      jj[u] = " << in.jx("i") << ";\n";
        if (with_val) l << "      xv[u] = " << in.xx("i") << ";\n";
        l << "    }\n"
          << "#pragma unroll\n"
          << "    for (int u = 0; u < 8; u++) {\n"
          << "      const bool in = i0 + u * 256 < hi;\n"
          << "      const int j = jj[u];\n"
          << body << "    }\n"
          << "  }\n";
        return l.str();
      };
      auto key_store = [&](const std::string &pos, const std::string &j) {
        return final_keys ? "keys[" + pos + "] = (unsigned short)(" + j + " & " + std::to_string(S - 1) + ");"
                          : "keys[" + pos + "] = " + j + ";";
      };
      std::string key_decl = final_keys ? "  unsigned short* const keys = (unsigned short*)b" + std::to_string(o.key) + ";\n"
                                        : "  int* const keys = b" + std::to_string(o.key) + ";\n";
      if (!local) {  // count: each wave into its own copy of the bucket
                     // counters (fewer same-address LDS atomics), the copies
                     // summed at the end
        int64_t NC = std::max<int64_t>(1, std::min<int64_t>(tune("scatter_count_copies", 4), 4));
        while (NC > 1 && NC * PB * 4 > 32768) NC /= 2;
        Params p = in.p;
        p.out.push_back(o.cnt);
        std::vector<int> args;
        std::string params = param_list(p, args);
        std::ostringstream k;
        k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "_count" << sfx << "(" << params << ") {\n"
          << "  __shared__ int lc[" << NC * PB << "];\n"
          << "  for (int q = threadIdx.x; q < " << NC * PB << "; q += 256) lc[q] = 0;\n"
          << "  __syncthreads();\n"
          << "  int* const mine = lc + (int)(threadIdx.x >> 6) % " << NC << " * " << PB << ";\n"
          << chunk_head()
          // 16 indices a thread per iteration in four 16-byte groups (lo is a
          // multiple of 256), the chunk's last partial group one by one
          << "  const int hi4 = lo + ((hi - lo) & ~3);\n"
          << "  for (int g0 = lo + 4 * (int)threadIdx.x; g0 < hi4; g0 += 4096) {\n"
          << "    int jj[16];\n"
          << "#pragma unroll\n"
          << "    for (int u = 0; u < 4; u++) {\n"
          << "      const int i = g0 + u * 1024 < hi4 ? g0 + u * 1024 : g0;\n"
          << "      " << in.vload_j("i") << "\n"
          << "      jj[4 * u] = " << in.jv("i", 0) << "; jj[4 * u + 1] = " << in.jv("i", 1) << ";\n"
          << "      jj[4 * u + 2] = " << in.jv("i", 2) << "; jj[4 * u + 3] = " << in.jv("i", 3) << ";\n"
          << "    }\n"
          << "#pragma unroll\n"
          << "    for (int u = 0; u < 16; u++) {\n"
          << "      const int j = jj[u];\n"
          << "      if (g0 + (u >> 2) * 1024 < hi4 && " << bounds("j") << ") cc_lds_add(&mine[j >> " << sh << "], 1);\n"
          << "    }\n"
          << "  }\n"
          << "  for (int i = hi4 + (int)threadIdx.x; i < hi; i += 256) {\n"
          << "    const int j = " << in.jx("i") << ";\n"
          << "    if (" << bounds("j") << ") cc_lds_add(&mine[j >> " << sh << "], 1);\n"
          << "  }\n"
          << "  __syncthreads();\n"
          << "  for (int q = threadIdx.x; q < " << PB << "; q += 256) {\n"
          << "    int c = lc[q];\n"
          << "    for (int w = 1; w < " << NC << "; w++) c += lc[w * " << PB << " + q];\n"
          << "    b" << o.cnt << "[(size_t)blockIdx.x * " << PB << " + q] = c;\n"
          << "  }\n"
          << "}\n";
        src << k.str();
        ks.push_back(add_kernel(kname + "_count" + sfx, args, (int)G, 256, "scatter_count"));
      }
      if (local) {
      } else if (PB >= 1024) {  // colscan, many buckets: a thread per bucket
                                // walks the chunks (loads coalesced across
                                // threads)
        std::ostringstream k;
        k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "_colscan" << sfx << "(int* __restrict__ b"
          << o.cnt << ", int* __restrict__ b" << o.start << ") {\n"
          << "  const int q = blockIdx.x * 256 + threadIdx.x;\n"
          << "  if (q >= " << PB << ") return;\n"
          << "  int run = 0;\n"
          << "  for (int c = 0; c < " << G << "; c++) {\n"
          << "    const int v = b" << o.cnt << "[(size_t)c * " << PB << " + q];\n"
          << "    b" << o.cnt << "[(size_t)c * " << PB << " + q] = run;\n"
          << "    run += v;\n"
          << "  }\n"
          << "  b" << o.start << "[q] = run;\n"
          << "}\n";
        src << k.str();
        ks.push_back(add_kernel(kname + "_colscan" + sfx, {o.cnt, o.start}, (int)cdiv(PB, 256), 256, "scatter_colscan"));
      } else {  // colscan, few buckets: one workgroup per bucket turns its
                // column of chunk counts into running offsets (each thread a
                // contiguous run of chunks, then a workgroup scan); start[q]
                // gets the bucket's total
        const int64_t per = cdiv(G, 256);
        std::ostringstream k;
        k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "_colscan" << sfx << "(int* __restrict__ b"
          << o.cnt << ", int* __restrict__ b" << o.start << ") {\n"
          << "  __shared__ int ws[4];\n"
          << "  const int q = blockIdx.x;\n"
          << "  const int c0 = threadIdx.x * " << per << ";\n"
          << "  int v[" << per << "], s = 0;\n"
          << "#pragma unroll\n"
          << "  for (int u = 0; u < " << per << "; u++) {\n"
          << "    v[u] = c0 + u < " << G << " ? b" << o.cnt << "[(size_t)(c0 + u) * " << PB << " + q] : 0;\n"
          << "    s += v[u];\n"
          << "  }\n"
          << "  int tot;\n"
          << "  int run = cc_wg_exscan(s, ws, &tot);\n"
          << "#pragma unroll\n"
          << "  for (int u = 0; u < " << per << "; u++)\n"
          << "    if (c0 + u < " << G << ") { b" << o.cnt << "[(size_t)(c0 + u) * " << PB << " + q] = run; run += v[u]; }\n"
          << "  if (threadIdx.x == 0) b" << o.start << "[q] = tot;\n"
          << "}\n";
        src << k.str();
        ks.push_back(add_kernel(kname + "_colscan" + sfx, {o.cnt, o.start}, (int)PB, 256, "scatter_colscan"));
      }
      if (!local) {  // bscan: one workgroup, exclusive prefix of the bucket totals
        int64_t per = cdiv(PB, 256);
        std::ostringstream k;
        k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "_bscan" << sfx << "(int* __restrict__ b"
          << o.start << ") {\n"
          << "  __shared__ int ps[257];\n"
          << "  const int lo = threadIdx.x * " << per << ";\n"
          << "  int s = 0;\n"
          << "  for (int q = lo; q < lo + " << per << " && q < " << PB << "; q++) s += b" << o.start << "[q];\n"
          << "  ps[threadIdx.x] = s;\n"
          << "  __syncthreads();\n"
          << "  if (threadIdx.x == 0) {\n"
          << "    int run = 0;\n"
          << "    for (int w = 0; w < 256; w++) { const int v = ps[w]; ps[w] = run; run += v; }\n"
          << "    ps[256] = run;\n"
          << "  }\n"
          << "  __syncthreads();\n"
          << "  int run = ps[threadIdx.x];\n"
          << "  for (int q = lo; q < lo + " << per << " && q < " << PB << "; q++) { const int v = b" << o.start
          << "[q]; b" << o.start << "[q] = run; run += v; }\n"
          << "  if (threadIdx.x == 0) b" << o.start << "[" << PB << "] = ps[256];\n"
          << "}\n";
        src << k.str();
        ks.push_back(add_kernel(kname + "_bscan" + sfx, {o.start}, 1, 256, "scatter_bscan"));
      }
      Params p = in.p;
      if (!local)
        for (int b : {o.cnt, o.start}) p.in.push_back(b);
      p.out.push_back(o.key);
      p.out.push_back(o.val);
      if (keep && staged) p.out.push_back(o.slot);
      if ((keep && staged) || local) p.out.push_back(o.meta);
      if (in.check) p.err = true;
      std::vector<int> args;
      std::string params = param_list(p, args);
      std::ostringstream k;
      // Threads of a staged partition workgroup (scatter_part_threads): its
      // LDS tile caps the workgroups per CU at two, so more threads per
      // workgroup keep more memory work in flight.
      const int64_t NT = staged ? part_threads : 256;
      const std::string snt = std::to_string(NT);
      k << "extern \"C\" __global__ __launch_bounds__(" << NT << ") void " << kname << "_partition" << sfx << "("
        << params << ") {\n";
      if (staged) {
        // each tile is grouped by bucket in LDS, then written as contiguous
        // runs
        const int64_t E = TILE / NT;
        int64_t PP = cdiv(PB, NT);
        if (local)
          // keys staged as 16 bits (the key within the slice), values beside
          k << "  __shared__ int tc[" << PB + 1 << "];\n"
            << "  __shared__ __align__(16) unsigned short sj[" << o.RS << "];\n"
            << "  __shared__ __align__(16) " << T << " sx[" << o.RS << "];\n"
            << "  __shared__ int ws[" << NT / 64 << "];\n"
            << "  int2* const runs = (int2*)b" << o.meta << ";\n"
            << key_decl << chunk_head();
        else
          k << "  __shared__ int cur[" << PB << "];\n"
            << "  __shared__ int tc[" << PB + 1 << "];\n"
            << "  __shared__ int sj[" << TILE << "];\n"
            << "  __shared__ " << T << " sx[" << TILE << "];\n"
            << "  __shared__ int ws[" << NT / 64 << "];\n"
            << "  for (int q = threadIdx.x; q < " << PB << "; q += " << NT << ") cur[q] = b" << o.start << "[q] + b"
            << o.cnt << "[(size_t)blockIdx.x * " << PB << " + q];\n"
            << key_decl << chunk_head();
        // The next tile's indices and values are loaded into a second set of
        // registers before this tile's LDS work starts (scatter_prefetch).
        const bool pf = tune("scatter_prefetch", 1) != 0;
        // A thread's E elements of a tile: E/4 groups of 4 consecutive
        // elements, group v at t + 4 NT v + 4 threadIdx.x (a multiple of 4:
        // tiles start at multiples of 256), each loaded with 16-byte
        // accesses; a group that runs past hi one by one, clamped.
        auto tile_load = [&](const std::string &t, const std::string &jv, const std::string &xvv) {
          std::ostringstream l;
          l << "#pragma unroll\n"
            << "    for (int v = 0; v < " << E / 4 << "; v++) {\n"
            << "      const int g = " << t << " + v * " << 4 * NT << " + 4 * (int)threadIdx.x;\n"
            << "      if (g + 4 <= hi) {\n"
            << "        " << in.vload_jx("g") << "\n";
          for (int kk = 0; kk < 4; kk++)
            l << "        " << jv << "[4 * v + " << kk << "] = " << in.jv("g", kk) << "; " << xvv << "[4 * v + " << kk
              << "] = " << in.xv("g", kk) << ";\n";
          l << "      } else {\n"
            << "#pragma unroll\n"
            << "        for (int c = 0; c < 4; c++) {\n"
            << "          const int i = g + c < hi ? g + c : lo;\n"
            << "          " << jv << "[4 * v + c] = " << in.jx("i") << ";\n"
            << "          " << xvv << "[4 * v + c] = " << in.xx("i") << ";\n"
            << "        }\n"
            << "      }\n"
            << "    }\n";
          return l.str();
        };
        // element u of the thread's tile (the layout above)
        const std::string eidx = "(t0 + (u >> 2) * " + std::to_string(4 * NT) + " + 4 * (int)threadIdx.x + (u & 3))";
        if (pf)
          k << "  int jn[" << E << "];\n"
            << "  " << T << " xn[" << E << "];\n"
            << "  if (lo < hi) {\n" << tile_load("lo", "jn", "xn") << "  }\n";
        k << "  for (int t0 = lo; t0 < hi; t0 += " << TILE << ") {\n";
        if (local) k << "    const int tt = blockIdx.x * " << o.TPC << " + (t0 - lo) / " << TILE << ";\n";
        k << "    for (int q = threadIdx.x; q < " << PB << "; q += " << NT << ") tc[q] = 0;\n"
          << "    int jj[" << E << "], rk[" << E << "];\n"
          << "    " << T << " xv[" << E << "];\n";
        if (pf)
          k << "#pragma unroll\n"
            << "    for (int u = 0; u < " << E << "; u++) { jj[u] = jn[u]; xv[u] = xn[u]; }\n"
            << "    if (t0 + " << TILE << " < hi) {\n" << tile_load("(t0 + " + std::to_string(TILE) + ")", "jn", "xn")
            << "    }\n";
        else
          k << tile_load("t0", "jj", "xv");
        k << "    __syncthreads();\n"
          << "#pragma unroll\n"
          << "    for (int u = 0; u < " << E << "; u++) {\n"
          << "      rk[u] = 0;\n"
          << "      if (" << eidx << " >= hi) { jj[u] = -1; continue; }\n"
          << "      if (" << bounds("jj[u]") << ") rk[u] = atomicAdd(&tc[jj[u] >> " << sh << "], 1);\n"
          << "      else { " << (in.check ? "cc_flag(err, 2); " : "") << "jj[u] = -1; }\n"
          << "    }\n"
          << "    __syncthreads();\n"
          << "    {\n";
        if (local)
          // runs padded to multiples of 8 elements; per bucket its run start
          // and count, and the region's used length
          k << "      int loc[" << PP << "], cn[" << PP << "], s = 0;\n"
            << "#pragma unroll\n"
            << "      for (int c = 0; c < " << PP << "; c++) {\n"
            << "        const int q = threadIdx.x * " << PP << " + c;\n"
            << "        loc[c] = s;\n"
            << "        cn[c] = q < " << PB << " ? tc[q] : 0;\n"
            << "        s += (cn[c] + 7) & ~7;\n"
            << "      }\n"
            << "      int tot;\n"
            << "      const int base = cc_wg_exscan_n<" << NT / 64 << ">(s, ws, &tot);\n"
            << "#pragma unroll\n"
            << "      for (int c = 0; c < " << PP << "; c++) {\n"
            << "        const int q = threadIdx.x * " << PP << " + c;\n"
            << "        if (q < " << PB << ") {\n"
            << "          tc[q] = base + loc[c];\n"
            << "          runs[(size_t)q * " << o.NTT << " + tt] = make_int2(base + loc[c], cn[c]);\n"
            << "        }\n"
            << "      }\n"
            << "      if (threadIdx.x == 0) {\n"
            << "        tc[" << PB << "] = tot;\n"
            << "        runs[(size_t)" << PB * o.NTT << " + tt] = make_int2(tot, 0);\n"
            << "      }\n";
        else if (!keep)
          k << "      int loc[" << PP << "], s = 0;\n"
            << "#pragma unroll\n"
            << "      for (int c = 0; c < " << PP << "; c++) {\n"
            << "        const int q = threadIdx.x * " << PP << " + c;\n"
            << "        loc[c] = s;\n"
            << "        s += q < " << PB << " ? tc[q] : 0;\n"
            << "      }\n"
            << "      int tot;\n"
            << "      const int base = cc_wg_exscan_n<" << NT / 64 << ">(s, ws, &tot);\n"
            << "#pragma unroll\n"
            << "      for (int c = 0; c < " << PP << "; c++) {\n"
            << "        const int q = threadIdx.x * " << PP << " + c;\n"
            << "        if (q < " << PB << ") tc[q] = base + loc[c];\n"
            << "      }\n"
            << "      if (threadIdx.x == 0) tc[" << PB << "] = tot;\n";
        else
          // The same scan also numbers the tile's non-empty buckets: the low
          // 16 bits carry the counts (a tile holds at most 8192 elements),
          // the high bits one per non-empty bucket (at most 4096). The
          // tile's record for the gather back: its number of non-empty
          // buckets K, their K tile-local starts and the tile's total, their
          // K run starts in the pair arrays.
          k << "      int loc[" << PP << "], cn[" << PP << "], s = 0;\n"
            << "#pragma unroll\n"
            << "      for (int c = 0; c < " << PP << "; c++) {\n"
            << "        const int q = threadIdx.x * " << PP << " + c;\n"
            << "        loc[c] = s;\n"
            << "        cn[c] = q < " << PB << " ? tc[q] : 0;\n"
            << "        s += cn[c] + (cn[c] > 0 ? 0x10000 : 0);\n"
            << "      }\n"
            << "      int tot;\n"
            << "      const int base = cc_wg_exscan_n<" << NT / 64 << ">(s, ws, &tot);\n"
            << "      const size_t mt = ((size_t)blockIdx.x * " << o.TPC << " + (t0 - lo) / " << TILE << ") * "
            << o.meta_stride() << ";\n"
            << "#pragma unroll\n"
            << "      for (int c = 0; c < " << PP << "; c++) {\n"
            << "        const int q = threadIdx.x * " << PP << " + c;\n"
            << "        const int pk = base + loc[c];\n"
            << "        if (q < " << PB << ") tc[q] = pk & 0xffff;\n"
            << "        if (cn[c] > 0) {\n"
            << "          b" << o.meta << "[mt + 1 + (pk >> 16)] = pk & 0xffff;\n"
            << "          b" << o.meta << "[mt + " << o.kmax() + 2 << " + (pk >> 16)] = cur[q];\n"
            << "        }\n"
            << "      }\n"
            << "      if (threadIdx.x == 0) {\n"
            << "        tc[" << PB << "] = tot & 0xffff;\n"
            << "        b" << o.meta << "[mt] = tot >> 16;\n"
            << "        b" << o.meta << "[mt + 1 + (tot >> 16)] = tot & 0xffff;\n"
            << "      }\n";
        k << "    }\n"
          << "    __syncthreads();\n";
        if (keep)
          k << "    {\n"
            << "      unsigned short* const slots = (unsigned short*)b" << o.slot << ";\n"

            // a group's four slots in one 8-byte store
            << "#pragma unroll\n"
            << "      for (int v = 0; v < " << E / 4 << "; v++) {\n"
            << "        const int g = t0 + v * " << 4 * NT << " + 4 * (int)threadIdx.x;\n"
            << "        unsigned sv[4];\n"
            << "#pragma unroll\n"
            << "        for (int c = 0; c < 4; c++)\n"
            << "          sv[c] = jj[4 * v + c] >= 0 ? (unsigned)(tc[jj[4 * v + c] >> " << sh << "] + rk[4 * v + c]) : 0xffffu;\n"
            << "        if (g + 4 <= hi) {\n"
            << "          *(uint2*)(slots + g) = make_uint2(sv[0] | (sv[1] << 16), sv[2] | (sv[3] << 16));\n"
            << "        } else {\n"
            << "#pragma unroll\n"
            << "          for (int c = 0; c < 4; c++) if (g + c < hi) slots[g + c] = (unsigned short)sv[c];\n"
            << "        }\n"
            << "      }\n"
            << "    }\n";
        if (local) {
          // the tile's region written whole, 8 elements a thread: one
          // 16-byte store of keys, 16-byte stores of values (padding
          // included; readers stop at each run's count)
          k << "#pragma unroll\n"
            << "    for (int u = 0; u < " << E << "; u++)\n"
            << "      if (jj[u] >= 0) {\n"
            << "        const int slot = tc[jj[u] >> " << sh << "] + rk[u];\n"
            << "        sj[slot] = (unsigned short)(jj[u] & " << S - 1 << ");\n"
            << "        sx[slot] = xv[u];\n"
            << "      }\n"
            << "    __syncthreads();\n"
            << "    {\n"
            << "      typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));\n"
            << "      typedef __attribute__((ext_vector_type(4))) " << T << " v4;\n"
            << "      const size_t rb = (size_t)tt * " << o.RS << ";\n"
            << "      for (int s = 8 * (int)threadIdx.x; s < tc[" << PB << "]; s += " << 8 * NT << ") {\n";
          if (tune("sp_nt", 0) & 2)
            k << "        __builtin_nontemporal_store(*(const u16x8*)(sj + s), (u16x8*)(keys + rb + s));\n"
              << "        __builtin_nontemporal_store(*(const v4*)(sx + s), (v4*)(b" << o.val << " + rb + s));\n"
              << "        __builtin_nontemporal_store(*(const v4*)(sx + s + 4), (v4*)(b" << o.val << " + rb + s + 4));\n";
          else
            k << "        *(u16x8*)(keys + rb + s) = *(const u16x8*)(sj + s);\n"
              << "        *(v4*)(b" << o.val << " + rb + s) = *(const v4*)(sx + s);\n"
              << "        *(v4*)(b" << o.val << " + rb + s + 4) = *(const v4*)(sx + s + 4);\n";
          k << "      }\n"
            << "    }\n"
            << "    __syncthreads();\n"
            << "  }\n"
            // a chunk's tiles past the end of the input: empty runs
            << "  for (int x = threadIdx.x + (hi - lo + " << TILE - 1 << ") / " << TILE << " * " << PB + 1 << "; x < "
            << o.TPC * (PB + 1) << "; x += " << NT << ")\n"
            << "    runs[(size_t)(x % " << PB + 1 << ") * " << o.NTT << " + blockIdx.x * " << o.TPC << " + x / "
            << PB + 1 << "] = make_int2(0, 0);\n";
        } else {
        k << "#pragma unroll\n"
          << "    for (int u = 0; u < " << E << "; u++)\n"
          << "      if (jj[u] >= 0) {\n"
          << "        const int slot = tc[jj[u] >> " << sh << "] + rk[u];\n"
          << "        sj[slot] = jj[u];\n"
          << "        sx[slot] = xv[u];\n"
          << "      }\n"
          << "    __syncthreads();\n"
          << "    for (int s = threadIdx.x; s < tc[" << PB << "]; s += " << NT << ") {\n"
          << "      const int j = sj[s], q = j >> " << sh << ";\n"
          << "      const int pos = cur[q] + (s - tc[q]);\n"
          << "      " << key_store("pos", "j") << "\n"
          << "      b" << o.val << "[pos] = sx[s];\n"
          << "    }\n"
          << "    __syncthreads();\n"
          << "    for (int q = threadIdx.x; q < " << PB << "; q += " << NT << ") cur[q] += tc[q + 1] - tc[q];\n"
          << "    __syncthreads();\n"
          << "  }\n";
        }
      } else {
        k << "  __shared__ int cur[" << PB << "];\n"
          << "  for (int q = threadIdx.x; q < " << PB << "; q += 256) cur[q] = b" << o.start << "[q] + b" << o.cnt
          << "[(size_t)blockIdx.x * " << PB << " + q];\n"
          << "  __syncthreads();\n"
          << key_decl << chunk_head()
          << loop8(true, "      if (in && " + bounds("j") + ") {\n"
                         "        const int pos = atomicAdd(&cur[j >> " + sh + "], 1);\n"
                         "        " + key_store("pos", "j") + "\n"
                         "        b" + std::to_string(o.val) + "[pos] = xv[u];\n"
                         "      }" + (in.check ? " else if (in) cc_flag(err, 2);" : "") + "\n");
      }
      k << "}\n";
      src << k.str();
      ks.push_back(add_kernel(kname + "_partition" + sfx, args, (int)G, (int)NT, part_role));
      return o;
    };

    // The slice pass of two levels in windows (PassOut::windows): one
    // workgroup per window of a super-slice's run in the coarse output,
    // grouped by its 64 slices into the window's own region, as a
    // tile-local pass does. No count or offset kernels.
    auto pass_windows = [&](const PassOut &c1, int64_t P1, bool keep_slots) {
      const int64_t TILE = 8192, NT = part_threads, E = TILE / NT;
      PassOut o;
      o.local = o.windows = true;
      o.wstart = c1.start;
      o.P1 = P1;
      o.PB = 64;
      o.TILE = TILE;
      o.first = false;
      o.NTT = cdiv(N, TILE) + P1;  // each super-slice adds at most one short window
      o.RS = TILE + 8 * 64;
      o.key = add_buf("t" + id + "_key", DT::I32, cdiv(o.NTT * o.RS, 2), BufRole::Scratch);  // 16-bit keys
      o.val = add_buf("t" + id + "_val", n.dt, o.NTT * o.RS, BufRole::Scratch);
      o.meta = add_buf("t" + id + "_runs", DT::I32, 2 * 65 * o.NTT, BufRole::Scratch);
      if (keep_slots) o.slot = add_buf("t" + id + "_slot", DT::I32, cdiv(N, 2), BufRole::Scratch);
      o.wtab = add_buf("t" + id + "_windows", DT::I32, P1 + 1, BufRole::Scratch);
      {  // each super-slice's first window: one wave, a prefix of window counts
        std::ostringstream k;
        k << "extern \"C\" __global__ __launch_bounds__(64) void " << kname << "_windows(const int* __restrict__ b"
          << c1.start << ", int* __restrict__ b" << o.wtab << ") {\n"
          // lane l takes super-slices [l PQ, l PQ + PQ)
          << "  const int l = threadIdx.x;\n"
          << "  int nt[" << cdiv(P1, 64) << "], sum = 0;\n"
          << "#pragma unroll\n"
          << "  for (int c = 0; c < " << cdiv(P1, 64) << "; c++) {\n"
          << "    const int Q = l * " << cdiv(P1, 64) << " + c;\n"
          << "    nt[c] = Q < " << P1 << " ? (b" << c1.start << "[Q + 1] - b" << c1.start << "[Q] + " << TILE - 1 << ") / "
          << TILE << " : 0;\n"
          << "    sum += nt[c];\n"
          << "  }\n"
          << "  int in = sum;\n"
          << "#pragma unroll\n"
          << "  for (int d = 1; d < 64; d <<= 1) {\n"
          << "    const int o_ = __shfl_up(in, d);\n"
          << "    if (l >= d) in += o_;\n"
          << "  }\n"
          << "  int run = in - sum;\n"
          << "#pragma unroll\n"
          << "  for (int c = 0; c < " << cdiv(P1, 64) << "; c++) {\n"
          << "    const int Q = l * " << cdiv(P1, 64) << " + c;\n"
          << "    if (Q < " << P1 << ") b" << o.wtab << "[Q] = run;\n"
          << "    run += nt[c];\n"
          << "  }\n"
          << "  if (l == 63) b" << o.wtab << "[" << P1 << "] = in;\n"
          << "}\n";
        src << k.str();
        ks.push_back(add_kernel(kname + "_windows", {c1.start, o.wtab}, 1, 64, "scatter_windows"));
      }
      std::vector<int> args = {c1.key, c1.val, c1.start, o.wtab, o.key, o.val, o.meta};
      if (keep_slots) args.push_back(o.slot);
      std::ostringstream k;
      k << "extern \"C\" __global__ __launch_bounds__(" << NT << ") void " << kname << "_partition(const int* __restrict__ b"
        << c1.key << ", const " << T << "* __restrict__ b" << c1.val << ", const int* __restrict__ b" << c1.start
        << ", const int* __restrict__ b" << o.wtab << ", int* __restrict__ b" << o.key << ", " << T
        << "* __restrict__ b" << o.val << ", int* __restrict__ b" << o.meta;
      if (keep_slots) k << ", int* __restrict__ b" << o.slot;
      k << ") {\n"
        << "  __shared__ int tc[65];\n"
        << "  __shared__ __align__(16) unsigned short sj[" << o.RS << "];\n"
        << "  __shared__ __align__(16) " << T << " sx[" << o.RS << "];\n"
        << "  int2* const runs = (int2*)b" << o.meta << ";\n"
        << "  unsigned short* const keys = (unsigned short*)b" << o.key << ";\n"
        << "  const int ft = blockIdx.x;\n"
        << window_at(o, "ft")
        << "  if (threadIdx.x < 64) tc[threadIdx.x] = 0;\n"
        << "  int jj[" << E << "], rk[" << E << "];\n"
        << "  " << T << " xv[" << E << "];\n"
        << "#pragma unroll\n"
        << "  for (int u = 0; u < " << E << "; u++) {\n"
        << "    const int i = (int)threadIdx.x + u * " << NT << ";\n"
        << "    jj[u] = i < wn_ ? b" << c1.key << "[wb_ + i] : -1;\n"
        << "    xv[u] = i < wn_ ? b" << c1.val << "[wb_ + i] : " << zero_of(n.dt) << ";\n"
        << "  }\n"
        << "  __syncthreads();\n"
        // the bin's slice within the super-slice (the coarse pass put only
        // this super-slice's bins here)
        << "#pragma unroll\n"
        << "  for (int u = 0; u < " << E << "; u++) rk[u] = jj[u] >= 0 ? atomicAdd(&tc[(jj[u] >> " << shift
        << ") & 63], 1) : 0;\n"
        << "  __syncthreads();\n"
        // one wave: runs padded to multiples of 8, their starts, and per
        // slice {start, count}; row 64 the region's used length
        << "  if (threadIdx.x < 64) {\n"
        << "    const int c = tc[threadIdx.x], pc = (c + 7) & ~7;\n"
        << "    int in = pc;\n"
        << "#pragma unroll\n"
        << "    for (int d = 1; d < 64; d <<= 1) {\n"
        << "      const int o_ = __shfl_up(in, d);\n"
        << "      if ((int)threadIdx.x >= d) in += o_;\n"
        << "    }\n"
        << "    tc[threadIdx.x] = in - pc;\n"
        << "    runs[(size_t)threadIdx.x * " << o.NTT << " + ft] = make_int2(in - pc, c);\n"
        << "    if (threadIdx.x == 63) {\n"
        << "      tc[64] = in;\n"
        << "      runs[(size_t)" << 64 * o.NTT << " + ft] = make_int2(in, 0);\n"
        << "    }\n"
        << "  }\n"
        << "  __syncthreads();\n"
        << "#pragma unroll\n"
        << "  for (int u = 0; u < " << E << "; u++)\n"
        << "    if (jj[u] >= 0) {\n"
        << "      const int slot = tc[(jj[u] >> " << shift << ") & 63] + rk[u];\n";
      if (keep_slots)
        k << "      ((unsigned short*)b" << o.slot << ")[wb_ + (int)threadIdx.x + u * " << NT
          << "] = (unsigned short)slot;\n";
      k << "      sj[slot] = (unsigned short)(jj[u] & " << S - 1 << ");\n"
        << "      sx[slot] = xv[u];\n"
        << "    }\n"
        << "  __syncthreads();\n"
        << "  typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));\n"
        << "  typedef __attribute__((ext_vector_type(4))) " << T << " v4;\n"
        << "  const size_t rb = (size_t)ft * " << o.RS << ";\n"
        << "  for (int s = 8 * (int)threadIdx.x; s < tc[64]; s += " << 8 * NT << ") {\n"
        << "    *(u16x8*)(keys + rb + s) = *(const u16x8*)(sj + s);\n"
        << "    *(v4*)(b" << o.val << " + rb + s) = *(const v4*)(sx + s);\n"
        << "    *(v4*)(b" << o.val << " + rb + s + 4) = *(const v4*)(sx + s + 4);\n"
        << "  }\n"
        << "}\n";
      src << k.str();
      ks.push_back(add_kernel(kname + "_partition", args, (int)o.NTT, (int)NT, "scatter_partition"));
      return o;
    };

    PassIn first;
    add_in(first.p, fi);
    add_in(first.p, fs);
    first.jx = [&](const std::string &i) { return fi.call_scalar(i); };
    first.xx = [&](const std::string &i) { return fs.call_scalar(i); };
    ElemFn fboth;  // identity loads shared by both functions, once
    fboth.ident = fi.ident;
    for (int b : fs.ident)
      if (std::find(fboth.ident.begin(), fboth.ident.end(), b) == fboth.ident.end()) fboth.ident.push_back(b);
    auto oneline = [](std::string t) {
      for (char &c : t)
        if (c == '\n') c = ' ';
      return t;
    };
    first.vload_j = [&, oneline](const std::string &i) { return oneline(vec_loads(fi, i, "", tyof())); };
    first.vload_jx = [&, oneline](const std::string &i) {
      return oneline(vec_loads(fboth, i, "", tyof(), (tune("sp_nt", 0) & 1) != 0));
    };
    first.jv = [&](const std::string &i, int k) { return lane_call(fi, i, k); };
    first.xv = [&](const std::string &i, int k) { return lane_call(fs, i, k); };
    first.nvalid = std::to_string(N);
    first.check = true;
    const int64_t STAGE_P = tune("scatter_stage_p", 512);
    // A gather back through this scatter's partition (a later root
    // gather(idx, h) over the same index) keeps the staged passes' slots.
    const bool keep = gbp_root_of.count(t) > 0;
    PassOut fin, coarse;
    // Tile-local layout up to 256 slices (runs of 32 elements a tile or
    // more, on average, for 8192-element tiles): scatter_local_max sets the
    // limit, 0 turns it off.
    const bool local = P <= tune("scatter_local_max", 256) && P <= STAGE_P;
    if (P <= STAGE_P) {
      fin = pass("", first, shift, P, true, true, "scatter_partition", keep, local);
    } else if (!tune("scatter_two_level", 1)) {
      // single level, element-wise stores
      fin = pass("", first, shift, P, false, true, "scatter_partition", false, false);
    } else {
      // Two levels: a coarse pass into super-slices of 64 slices (runs of
      // about 64 elements per tile), then the slice pass over the coarse
      // output, whose tiles each touch at most two super-slices.
      const int64_t P1 = cdiv(P, 64);
      PassOut c1 = pass("1", first, shift + 6, P1, true, false, "scatter_coarse", keep, false);
      coarse = c1;
      if (tune("scatter_windows", 1)) {
        // the slice pass in windows of each super-slice's run
        fin = pass_windows(c1, P1, keep);
      } else {
      PassIn second;
      for (int b : {c1.key, c1.val, c1.start}) second.p.in.push_back(b);
      second.jx = [&, c1](const std::string &i) { return "b" + std::to_string(c1.key) + "[" + i + "]"; };
      second.xx = [&, c1](const std::string &i) { return "b" + std::to_string(c1.val) + "[" + i + "]"; };
      const std::string kb = "b" + std::to_string(c1.key), vb = "b" + std::to_string(c1.val);
      second.vload_j = [kb](const std::string &i) {
        return "const cc_v4<int> lk_ = *(const cc_v4<int>*)(" + kb + " + " + i + ");";
      };
      second.vload_jx = [kb, vb, T](const std::string &i) {
        return "const cc_v4<int> lk_ = *(const cc_v4<int>*)(" + kb + " + " + i + "); const cc_v4<" + T +
               "> lv_ = *(const cc_v4<" + T + ">*)(" + vb + " + " + i + ");";
      };
      second.jv = [](const std::string &, int k) { return std::string("lk_.") + "xyzw"[k]; };
      second.xv = [](const std::string &, int k) { return std::string("lv_.") + "xyzw"[k]; };
      second.nvalid = "b" + std::to_string(c1.start) + "[" + std::to_string(P1) + "]";
      second.nbuf = c1.start;
      second.check = false;
      fin = pass("", second, shift, P, true, true, "scatter_partition", keep, false);
      }
    }
    if (keep && fin.slot >= 0) {
      GatherBack gb;
      gb.fin = fin;
      gb.coarse = coarse;
      gb.S = S;
      gb.P = P;
      gb.B = B;
      gb.N = N;
      gb.h = out;
      gather_back[t] = gb;
    }
    const int start = fin.start, key = fin.key, val = fin.val;
    {  // accumulate
      int dst = part >= 0 ? part : out;
      // Threads per workgroup: the LDS table caps the workgroups per CU, so
      // more threads keep more loads in flight. 1024 where a slice has
      // several workgroups (config 3: 0.545 ms a step against 0.552 with
      // 512), 512 where it has one, whose workgroups are short (config 3b:
      // 1.071 against 1.104 ms); scatter_acc_threads=256, 512 or 1024
      // forces one.
      const int64_t at_default = W == 1 ? 512 : 1024;
      const int64_t AT = tune("scatter_acc_threads", at_default) == 256    ? 256
                         : tune("scatter_acc_threads", at_default) == 512  ? 512
                         : tune("scatter_acc_threads", at_default) == 1024 ? 1024
                                                                           : at_default;
      const int lead = fin.local ? fin.meta : start;  // where the slice's pairs are found
      // With one workgroup a slice its table is final in LDS at the end, so
      // a gather back's slice step (each pair's value replaced by h at its
      // bin) runs here, in a second walk over the same pairs.
      const bool fuse_back = W == 1 && gather_back.count(t) > 0 && tune("scatter_fuse_back", 1) != 0;
      if (fuse_back) gather_back[t].fused = true;
      // groups of 8 pairs a lane keeps in flight in the walks over the runs
      const int64_t acc_groups = std::max<int64_t>(1, std::min<int64_t>(8, tune("acc_groups", 2)));
      const int64_t back_groups = std::max<int64_t>(1, std::min<int64_t>(8, tune("gb_groups", 2)));
      std::ostringstream k;
      k << "extern \"C\" __global__ __launch_bounds__(" << AT << ") void " << kname << "_accumulate(const int* __restrict__ b"
        << lead << ", const int* __restrict__ b" << key << ", " << (fuse_back ? "" : "const ") << T << "* __restrict__ b"
        << val << ", " << T << "* __restrict__ b" << dst;
      if (fin.windows) k << ", const int* __restrict__ b" << fin.wtab;
      // the table cleared and stored 4 bins at a time (S is a multiple of 4;
      // a table cut short by the end of the bins stores its tail one by one)
      const std::string tv4 = "__attribute__((ext_vector_type(4))) " + T;
      k << ") {\n"
        << "  __shared__ __align__(16) " << T << " h[" << S << "];\n"
        << "  const int q = blockIdx.x / " << W << ", w = blockIdx.x % " << W << ";\n"
        << "  for (int b = 4 * (int)threadIdx.x; b < " << S << "; b += " << 4 * AT << ") *(" << tv4 << "*)(h + b) = ("
        << tv4 << ")" << zero_of(n.dt) << ";\n"
        << "  __syncthreads();\n";
      if (fin.local) {
        // the slice's runs in W shares of the tiles; a group's elements past
        // its run's count add +0 into bin 0 (see below)
        const std::string z = zero_of(n.dt);
        if (fin.windows)  // the windows of the slice's super-slice
          k << windows_of(fin, "(q >> 6)")
            << "  const int t_lo = ta_ + (int)((long long)(tz_ - ta_) * w / " << W << ");\n"
            << "  const int t_hi = ta_ + (int)((long long)(tz_ - ta_) * (w + 1) / " << W << ");\n";
        else
          k << "  const int t_lo = (int)((long long)" << fin.NTT << " * w / " << W << ");\n"
            << "  const int t_hi = (int)((long long)" << fin.NTT << " * (w + 1) / " << W << ");\n";
        k << "  const unsigned short* const keys = (const unsigned short*)b" << key << ";\n"
          << "  const " << T << "* const vals = b" << val << ";\n"
          << "  typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));\n"
          << "  typedef __attribute__((ext_vector_type(4))) " << T << " v4;\n"
          << runs_walk(fin, AT, fin.windows ? cdiv(cdiv(N, fin.TILE), fin.P1) / W : fin.NTT / W,
                       "        u16x8 kv[UG_];\n"
                       "        v4 xa[UG_], xb[UG_];\n"
                       "#pragma unroll\n"
                       "        for (int u = 0; u < UG_; u++) {\n" +
                       std::string(tune("acc_nt", 0) ?
                       "          kv[u] = __builtin_nontemporal_load((const u16x8*)(keys + pos_[u]));\n"
                       "          xa[u] = __builtin_nontemporal_load((const v4*)(vals + pos_[u]));\n"
                       "          xb[u] = __builtin_nontemporal_load((const v4*)(vals + pos_[u] + 4));\n" :
                       "          kv[u] = *(const u16x8*)(keys + pos_[u]);\n"
                       "          xa[u] = *(const v4*)(vals + pos_[u]);\n"
                       "          xb[u] = *(const v4*)(vals + pos_[u] + 4);\n") +
                       "        }\n",
                       "#pragma unroll\n"
                       "        for (int u = 0; u < UG_; u++)\n"
                       "#pragma unroll\n"
                       "          for (int e = 0; e < 8; e++) {\n"
                       "            const bool in = e < nv_[u];\n"
                       "            cc_lds_add(&h[in ? kv[u][e] : 0], in ? (e < 4 ? xa[u][e] : xb[u][e - 4]) : " + z + ");\n"
                       "          }\n", acc_groups)
          << "  __syncthreads();\n";
        if (fuse_back)
          k << "  " << T << "* const valw = b" << val << ";\n"
            << runs_walk(fin, AT, fin.windows ? cdiv(cdiv(N, fin.TILE), fin.P1) / W : fin.NTT / W,
                         "        u16x8 kv[UG_];\n"
                         "#pragma unroll\n"
                         "        for (int u = 0; u < UG_; u++) kv[u] = *(const u16x8*)(keys + pos_[u]);\n",
                         "#pragma unroll\n"
                         "        for (int u = 0; u < UG_; u++)\n"
                         "          if (nv_[u] > 0) {\n"
                         "            " + T + " x[8];\n"
                         "#pragma unroll\n"
                         "            for (int e = 0; e < 8; e++) x[e] = h[e < nv_[u] ? kv[u][e] : 0];\n"
                         "            *(v4*)(valw + pos_[u]) = (v4){x[0], x[1], x[2], x[3]};\n"
                         "            *(v4*)(valw + pos_[u] + 4) = (v4){x[4], x[5], x[6], x[7]};\n"
                         "          }\n", back_groups);
      } else {
      k << "  const int s0 = b" << start << "[q], len = b" << start << "[q + 1] - s0;\n"
        << "  const int lo = s0 + (int)((long long)len * w / " << W << ");\n"
        << "  const int hi = s0 + (int)((long long)len * (w + 1) / " << W << ");\n"
        << "  const unsigned short* const keys = (const unsigned short*)b" << key << ";\n"
        << "  const " << T << "* const vals = b" << val << ";\n"
        // the 8-aligned body: 8 keys in one 16-byte load and 8 values in
        // 16-byte vectors, two groups a thread in flight; the unaligned head
        // and tail one by one
        << "  typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));\n"
        << "  typedef __attribute__((ext_vector_type(4))) " << T << " v4;\n"
        << "  const int up8 = (lo + 7) & ~7, dn8 = hi & ~7;\n"
        << "  const int lo8 = up8 < hi ? up8 : hi;\n"
        << "  const int hi8 = dn8 > lo8 ? dn8 : lo8;\n"
        << "  for (int i = lo + (int)threadIdx.x; i < lo8; i += " << AT << ") cc_lds_add(&h[keys[i]], vals[i]);\n"
        << "  for (int i = hi8 + (int)threadIdx.x; i < hi; i += " << AT << ") cc_lds_add(&h[keys[i]], vals[i]);\n"
        << "  for (int j0 = lo8 + 8 * (int)threadIdx.x; j0 < hi8; j0 += " << 16 * AT << ") {\n"
        << "    u16x8 kv[2];\n"
        << "    v4 xa[2], xb[2];\n"
        << "#pragma unroll\n"
        << "    for (int u = 0; u < 2; u++) {\n"
        << "      const int j = j0 + u * " << 8 * AT << " < hi8 ? j0 + u * " << 8 * AT << " : j0;\n"
        << "      kv[u] = *(const u16x8*)(keys + j);\n"
        << "      xa[u] = *(const v4*)(vals + j);\n"
        << "      xb[u] = *(const v4*)(vals + j + 4);\n"
        << "    }\n"
        // a group past the end adds +0 into bin 0, which leaves every bin
        // unchanged (tables start at +0, so no bin holds -0) and keeps the
        // use of the loads unconditional
        << "#pragma unroll\n"
        << "    for (int u = 0; u < 2; u++) {\n"
        << "      const bool in = j0 + u * " << 8 * AT << " < hi8;\n"
        << "#pragma unroll\n"
        << "      for (int e = 0; e < 8; e++)\n"
        << "        cc_lds_add(&h[in ? kv[u][e] : 0], in ? (e < 4 ? xa[u][e] : xb[u][e - 4]) : " << zero_of(n.dt) << ");\n"
        << "    }\n"
        << "  }\n"
        << "  __syncthreads();\n";
      if (fuse_back)
        k << "  " << T << "* const valw = b" << val << ";\n"
          << "  for (int i = lo + (int)threadIdx.x; i < lo8; i += " << AT << ") valw[i] = h[keys[i]];\n"
          << "  for (int i = hi8 + (int)threadIdx.x; i < hi; i += " << AT << ") valw[i] = h[keys[i]];\n"
          << "  for (int j0 = lo8 + 8 * (int)threadIdx.x; j0 < hi8; j0 += " << 8 * AT << ") {\n"
          << "    const u16x8 kv = *(const u16x8*)(keys + j0);\n"
          << "    *(v4*)(valw + j0) = (v4){h[kv[0]], h[kv[1]], h[kv[2]], h[kv[3]]};\n"
          << "    *(v4*)(valw + j0 + 4) = (v4){h[kv[4]], h[kv[5]], h[kv[6]], h[kv[7]]};\n"
          << "  }\n";
      }
      if (part >= 0)
        k << "  for (int b = 4 * (int)threadIdx.x; b < " << S << "; b += " << 4 * AT << ") *(" << tv4 << "*)(b" << dst
          << " + (size_t)w * " << P * S << " + (size_t)q * " << S << " + b) = *(const " << tv4 << "*)(h + b);\n";
      else
        k << "  const int nb = " << B << " - q * " << S << " < " << S << " ? " << B << " - q * " << S << " : " << S
          << ";\n"
          << "  for (int b = 4 * (int)threadIdx.x; b < nb; b += " << 4 * AT << ") {\n"
          << "    if (b + 4 <= nb) *(" << tv4 << "*)(b" << dst << " + (size_t)q * " << S << " + b) = *(const " << tv4
          << "*)(h + b);\n"
          << "    else for (int e = b; e < nb; e++) b" << dst << "[(size_t)q * " << S << " + e] = h[e];\n"
          << "  }\n";
      k << "}\n";
      src << k.str();
      std::vector<int> aargs = {lead, key, val, dst};
      if (fin.windows) aargs.push_back(fin.wtab);
      ks.push_back(add_kernel(kname + "_accumulate", aargs, (int)(P * W), (int)AT, "scatter_accumulate"));
    }
    if (part >= 0) ks.push_back(scatter_reduce(kname, T, acc, part, out, W, B, P * S));
    return ks;
  }

  // out[b] = sum over w of part[w * stride + b], w ascending.
  int scatter_reduce(const std::string &kname, const std::string &T, const std::string &acc, int part, int out,
                     int64_t W, int64_t B, int64_t stride) {
    std::ostringstream k;
    k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "_reduce(const " << T
      << "* __restrict__ b" << part << ", " << T << "* __restrict__ b" << out << ") {\n"
      << "  for (int b = blockIdx.x * 256 + threadIdx.x; b < " << B << "; b += gridDim.x * 256) {\n"
      << "    " << acc << " s = (" << acc << ")b" << part << "[b];\n"
      << "    for (int w = 1; w < " << W << "; w++) s += (" << acc << ")b" << part << "[(size_t)w * " << stride
      << " + b];\n"
      << "    b" << out << "[b] = (" << T << ")s;\n"
      << "  }\n"
      << "}\n";
    src << k.str();
    return add_kernel(kname + "_reduce", {part, out}, (int)std::min<int64_t>(cdiv(B, 256), 4096), 256,
                      "scatter_reduce");
  }

  // An i32 tensor that is exactly a*i + b in its flat element index i:
  // integer +, - and * by a constant over iota, the map's element index and
  // constants, through maps and reshapes. Wrapping i32 arithmetic agrees
  // with the exact value modulo 2^32, so where the exact value lies in
  // [0, 2^31) it is the value the reference computes.
  struct Aff {
    bool ok = false;
    int64_t a = 0, b = 0;
  };
  static bool aff_small(int64_t v) { return v > -(int64_t(1) << 40) && v < (int64_t(1) << 40); }
  Aff aff_x(int x, const std::vector<Aff> &args) const {
    const XNode &e = g.xs[x];
    if (e.dt != DT::I32) return {};
    switch (e.kind) {
      case XK::Const: return {true, 0, e.i};
      case XK::Arg: return e.arg < (int)args.size() ? args[e.arg] : Aff{};
      case XK::Index: return {true, 1, 0};
      case XK::Bin: {
        const Aff l = aff_x(e.a, args), r = aff_x(e.b, args);
        if (!l.ok || !r.ok) return {};
        Aff o;
        o.ok = true;
        if (e.op == B_ADD) {
          o.a = l.a + r.a;
          o.b = l.b + r.b;
        } else if (e.op == B_SUB) {
          o.a = l.a - r.a;
          o.b = l.b - r.b;
        } else if (e.op == B_MUL && (l.a == 0 || r.a == 0)) {
          const Aff &c = l.a == 0 ? l : r, &v = l.a == 0 ? r : l;
          if (__builtin_mul_overflow(c.b, v.a, &o.a) || __builtin_mul_overflow(c.b, v.b, &o.b)) return {};
        } else {
          return {};
        }
        return aff_small(o.a) && aff_small(o.b) ? o : Aff{};
      }
      default: return {};
    }
  }
  Aff aff_t(int t) const {
    const TNode &n = g.ts[t];
    if (n.dt != DT::I32) return {};
    switch (n.kind) {
      case TK::Iota: return {true, 1, 0};
      case TK::Reshape: return aff_t(n.a);
      case TK::Map: return aff_x(n.body, {aff_t(n.a)});
      case TK::Map2: return aff_x(n.body, {aff_t(n.a), aff_t(n.b)});
      default: return {};
    }
  }

  std::vector<int> lower_scatter(int t) {
    const TNode &n = g.ts[t];
    std::string id = std::to_string(n.id);
    std::string kname = "k_" + id;
    std::string T = dt_ctype(n.dt);
    int out = buf_of[t];
    int64_t M = n.numel;
    int64_t N = g.ts[n.a].numel;
    // An index a*i + b with a != 0 and every value in range hits each bin
    // at most once (the adjoint of a strided gather, such as the last
    // column of the path matrix): then each bin is 0 + its one source
    // value or 0, written by one pass over the bins, with no atomics and no
    // partition (scatter_affine=0 turns this off).
    const Aff ia = aff_t(n.a);
    if (ia.ok && ia.a != 0 && M > 0 && N > 0 && tune("scatter_affine", 1)) {
      const __int128 e0 = ia.b, e1 = (__int128)ia.a * (N - 1) + ia.b;
      if (std::min(e0, e1) >= 0 && std::max(e0, e1) < M) return lower_scatter_affine(t, ia.a, ia.b);
    }
    if (M > 0 && N > 0 && tune("scatter_lds", 1)) {
      const int64_t ES = dt_size(n.dt);
      // Slices of 16384 bins where the table fits 64 KiB of LDS (8192 for
      // 8-byte types): the longer a slice, the longer each tile's run of it
      // (config 3, 2^20 bins: 640 -> 614 us against 8192). A table of 128
      // KiB a workgroup (scatter_slice_lds=131072) is allowed too.
      const int64_t lds = tune("scatter_slice_lds", 65536) == 131072 ? 131072 : 65536;
      int64_t S = 4096;
      const int64_t want = tune("scatter_slice_bins", 16384);
      while (S < want && S * 2 * ES <= lds) S *= 2;
      while (cdiv(M, S) > 4096 && S * ES < lds) S *= 2;
      int64_t P = cdiv(M, S);
      // Two levels with the slice pass in windows take up to 8192 slices
      // (128 super-slices); the counted forms up to 4096.
      const bool windows = P > tune("scatter_stage_p", 512) && tune("scatter_two_level", 1) && tune("scatter_windows", 1);
      if (P == 1) return lower_scatter_lds(t, M, N, M, 1);
      if (P <= 4096 || (windows && P <= 8192)) return lower_scatter_lds(t, M, N, S, P);
    }
    std::vector<int> ks;
    if (M > 0) {
      // 16-byte stores, one group a lane over a grid as wide as the table
      // (the map template's shape), the ragged tail by the first lanes
      const int ZG = dt_size(n.dt) == 8 ? 2 : 4;
      const int64_t zvec = M / ZG;
      std::ostringstream z;
      z << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "_zero(" << T << "* __restrict__ b"
        << out << ") {\n"
        << "  typedef " << T << " zv __attribute__((ext_vector_type(" << ZG << ")));\n"
        << "  for (long long v = (long long)blockIdx.x * 256 + threadIdx.x; v < " << zvec
        << "; v += (long long)gridDim.x * 256) ((zv*)b" << out << ")[v] = (zv)(" << zero_of(n.dt) << ");\n"
        << "  if (blockIdx.x == 0 && (long long)threadIdx.x < " << M - zvec * ZG << ") b" << out << "[" << zvec * ZG
        << " + threadIdx.x] = " << zero_of(n.dt) << ";\n}\n";
      src << z.str();
      ks.push_back(add_kernel(kname + "_zero", {out}, (int)std::min<int64_t>(std::max<int64_t>(1, cdiv(zvec, 256)), 1 << 22),
                              256, "scatter_zero"));
    }
    if (N == 0) return ks;
    ElemFn fi = gen.element_fn("fi_" + id, n.a, false, true);
    ElemFn fs = gen.element_fn("fs_" + id, n.b, false, true);
    src << fi.code << fs.code;
    Params p;
    add_in(p, fi);
    add_in(p, fs);
    p.out.push_back(out);
    p.err = true;
    std::vector<int> args;
    std::string params = param_list(p, args);
    // Identity loads shared by both functions are loaded once.
    ElemFn both;
    both.ident = fi.ident;
    for (int b : fs.ident) {
      bool dup = false;
      for (int x : both.ident) dup |= x == b;
      if (!dup) both.ident.push_back(b);
    }
    std::ostringstream k;
    k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "(" << params << ") {\n"
      << "  const int stride = gridDim.x * 256;\n"
      << "  const int nvec = " << N / 4 << ";\n"
      << "  for (int v = blockIdx.x * 256 + threadIdx.x; v < nvec; v += stride) {\n"
      << "    const int i = v * 4;\n"
      << vec_loads(both, "i", "    ", tyof());
    for (int u = 0; u < 4; u++)
      k << "    { const int j = " << lane_call(fi, "i", u) << "; const " << T << " x = " << lane_call(fs, "i", u)
        << ";\n      if ((unsigned)j < " << M << "u) cc_atomic_add(b" << out << " + j, x); else cc_flag(err, 2); }\n";
    k << "  }\n"
      << "  for (int i = nvec * 4 + blockIdx.x * 256 + threadIdx.x; i < " << N << "; i += stride) {\n"
      << "    const int j = " << fi.call_scalar("i") << "; const " << T << " x = " << fs.call_scalar("i") << ";\n"
      << "    if ((unsigned)j < " << M << "u) cc_atomic_add(b" << out << " + j, x); else cc_flag(err, 2);\n"
      << "  }\n}\n";
    src << k.str();
    int64_t nvec = std::max<int64_t>(1, N / 4);
    ks.push_back(add_kernel(kname, args, (int)std::min<int64_t>(cdiv(nvec, 256), 1 << 22), 256, "scatter_atomic"));
    return ks;
  }

  // scatter_add with an injective affine index (see lower_scatter): one
  // pass over the bins, four a thread on a grid as wide as the table, each
  // bin j taking
  // 0 + src((j - b) / a) where a divides j - b and the quotient is a source
  // index, else 0.
  std::vector<int> lower_scatter_affine(int t, int64_t A, int64_t Bc) {
    const TNode &n = g.ts[t];
    const std::string id = std::to_string(n.id), kname = "k_" + id, T = dt_ctype(n.dt);
    const int out = buf_of[t];
    const int64_t M = n.numel, N = g.ts[n.a].numel;
    ElemFn fs = gen.element_fn("fs_" + id, n.b, false, true);
    src << fs.code;
    Params p;
    add_in(p, fs);
    p.out.push_back(out);
    std::vector<int> args;
    std::string params = param_list(p, args);
    const bool wide = M > INT32_MAX - 4 || Bc > INT32_MAX || Bc < INT32_MIN || A > INT32_MAX || A < INT32_MIN;
    const std::string I = wide ? "long long" : "int";
    const std::string z = zero_of(n.dt);
    std::ostringstream k;
    k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "_affine(" << params << ") {\n"
      << "  for (" << I << " j0 = 4 * ((" << I << ")blockIdx.x * 256 + threadIdx.x); j0 < " << M << "; j0 += 4 * ("
      << I << ")gridDim.x * 256) {\n"
      << "    " << T << " v[4];\n"
      << "#pragma unroll\n"
      << "    for (int u = 0; u < 4; u++) {\n"
      << "      const " << I << " q = j0 + u - (" << Bc << ");\n"
      << "      v[u] = " << z << ";\n"
      << "      if (q % (" << A << ") == 0) {\n"
      << "        const " << I << " i = q / (" << A << ");\n"
      << "        if (i >= 0 && i < " << N << ") v[u] = " << z << " + " << fs.call_scalar("(int)i") << ";\n"
      << "      }\n"
      << "    }\n"
      << "    if (j0 + 4 <= " << M << ") {\n";
    // streamed past the caches where the table is larger than the MALL
    if (streams(M * dt_size(n.dt)))
      k << "      cc_st4_nt(b" << out << " + j0, cc_v4<" << T << ">{v[0], v[1], v[2], v[3]});\n";
    else
      k << "      *(__attribute__((ext_vector_type(4))) " << T << "*)(b" << out
        << " + j0) = (__attribute__((ext_vector_type(4))) " << T << "){v[0], v[1], v[2], v[3]};\n";
    k << "    } else {\n"
      << "      for (int u = 0; j0 + u < " << M << "; u++) b" << out << "[j0 + u] = v[u];\n"
      << "    }\n"
      << "  }\n"
      << "}\n";
    src << k.str();
    return {add_kernel(kname + "_affine", args, (int)std::min<int64_t>(cdiv(cdiv(M, 4), 256), tune("map_blocks", 1 << 22)), 256,
                       "scatter_affine")};
  }

  // ---- Gather back through a scatter's partition ----------------------------
  // back = gather(idx, h) with h = scatter_add(idx, src, bins) lowered through
  // the LDS partition: the partition already grouped the index stream by
  // table slice, so the gather reads the table slice by slice from LDS
  // instead of making one random L2 request per element (config 3's
  // 4 MiB-table gather sits at the L2 request ceiling; a 256 MiB table
  // fetches one HBM line per element).
  //   slices      each pair's value becomes h at its bin, from an LDS copy
  //               of its slice (in place, in pair order; the pairs' values
  //               are dead once accumulated)
  //   unpartition per tile of a pass: the tile's runs staged through LDS in
  //               its bucket-grouped order, then each element takes the
  //               value at its recorded slot; two-level partitions are
  //               undone level by level
  // An element the scatter skipped (index out of range) has no slot: it
  // gets zero and raises the gather's error, as the gather would.
  std::vector<int> lower_gather_back(int r, const GatherBack &gb) {
    const TNode &n = g.ts[r];
    const std::string kname = "k_" + std::to_string(n.id);
    const std::string T = dt_ctype(n.dt);
    const int out = buf_of[r];
    const PassOut &f = gb.fin;
    std::vector<int> ks;
    // 8 values of T through 16-byte accesses: two 4-wide vectors
    const std::string v4 = "__attribute__((ext_vector_type(4))) " + T;
    // Threads per workgroup of both kernels, whose LDS caps the workgroups
    // per CU: 512 (config 3's unpartition 184 -> 154 us; config 3b's slices
    // 161 -> 131, unpartition passes 224 / 172 -> 168 / 143 us, against
    // 256; 1024 is in between); gather_threads=256 or 1024 for the others.
    const int64_t GT = tune("gather_threads", 512) == 256 ? 256 : tune("gather_threads", 512) == 1024 ? 1024 : 512;
    if (!gb.fused) {  // (otherwise the accumulate did this step)
      const int64_t S = gb.S, B = gb.B;
      const int64_t Wg = std::max<int64_t>(1, std::min<int64_t>(16, 1024 / gb.P));
      const int lead = f.local ? f.meta : f.start;  // where each slice's pairs are found
      std::ostringstream k;
      k << "extern \"C\" __global__ __launch_bounds__(" << GT << ") void " << kname << "_slices(const int* __restrict__ b"
        << lead << ", const int* __restrict__ b" << f.key << ", const " << T << "* __restrict__ b" << gb.h << ", "
        << T << "* __restrict__ b" << f.val;
      if (f.windows) k << ", const int* __restrict__ b" << f.wtab;
      k << ") {\n"
        << "  typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));\n"
        << "  typedef " << v4 << " v4;\n"
        << "  __shared__ " << T << " tab[" << S << "];\n"
        << "  const int q = blockIdx.x / " << Wg << ", w = blockIdx.x % " << Wg << ";\n"
        << "  const int nb = " << B << " - q * " << S << " < " << S << " ? " << B << " - q * " << S << " : " << S
        << ";\n"
        << "  const " << T << "* const hq = b" << gb.h << " + (size_t)q * " << S << ";\n"
        // the slice into LDS, eight loads in flight per thread
        << "  for (int b0 = threadIdx.x; b0 < nb; b0 += " << 8 * GT << ") {\n"
        << "    " << T << " t[8];\n"
        << "#pragma unroll\n"
        << "    for (int u = 0; u < 8; u++) t[u] = hq[b0 + u * " << GT << " < nb ? b0 + u * " << GT << " : b0];\n"
        << "#pragma unroll\n"
        << "    for (int u = 0; u < 8; u++) if (b0 + u * " << GT << " < nb) tab[b0 + u * " << GT << "] = t[u];\n"
        << "  }\n"
        << "  __syncthreads();\n";
      if (f.local) {
        // the slice's runs in Wg shares of the tiles; a group's elements past
        // its run's count read bin 0 and land in the run's padding
        if (f.windows)  // the windows of the slice's super-slice
          k << windows_of(f, "(q >> 6)")
            << "  const int t_lo = ta_ + (int)((long long)(tz_ - ta_) * w / " << Wg << ");\n"
            << "  const int t_hi = ta_ + (int)((long long)(tz_ - ta_) * (w + 1) / " << Wg << ");\n";
        else
          k << "  const int t_lo = (int)((long long)" << f.NTT << " * w / " << Wg << ");\n"
            << "  const int t_hi = (int)((long long)" << f.NTT << " * (w + 1) / " << Wg << ");\n";
        k << "  const unsigned short* const keys = (const unsigned short*)b" << f.key << ";\n"
          << "  " << T << "* const vals = b" << f.val << ";\n"
          << runs_walk(f, GT, f.windows ? cdiv(cdiv(gb.N, f.TILE), f.P1) / Wg : f.NTT / Wg,
                       "        u16x8 kv[UG_];\n"
                       "#pragma unroll\n" +
                           std::string("        for (int u = 0; u < UG_; u++) kv[u] = ") +
                           ((tune("gs_nt", 0) & 2) ? "__builtin_nontemporal_load((const u16x8*)(keys + pos_[u]));\n"
                                                   : "*(const u16x8*)(keys + pos_[u]);\n"),
                       "#pragma unroll\n"
                       "        for (int u = 0; u < UG_; u++)\n"
                       "          if (nv_[u] > 0) {\n"
                       "            " + T + " x[8];\n"
                       "#pragma unroll\n"
                       "            for (int e = 0; e < 8; e++) x[e] = tab[e < nv_[u] ? kv[u][e] : 0];\n"
                       + std::string((tune("gs_nt", 0) & 1)
                           ? "            __builtin_nontemporal_store((v4){x[0], x[1], x[2], x[3]}, (v4*)(vals + pos_[u]));\n"
                             "            __builtin_nontemporal_store((v4){x[4], x[5], x[6], x[7]}, (v4*)(vals + pos_[u] + 4));\n"
                           : "            *(v4*)(vals + pos_[u]) = (v4){x[0], x[1], x[2], x[3]};\n"
                             "            *(v4*)(vals + pos_[u] + 4) = (v4){x[4], x[5], x[6], x[7]};\n") +
                       "          }\n", tune("gb_groups", 2))
          << "}\n";
      } else {
      k << "  const int s0 = b" << f.start << "[q], len = b" << f.start << "[q + 1] - s0;\n"
        << "  const int lo = s0 + (int)((long long)len * w / " << Wg << ");\n"
        << "  const int hi = s0 + (int)((long long)len * (w + 1) / " << Wg << ");\n"
        << "  const unsigned short* const keys = (const unsigned short*)b" << f.key << ";\n"
        << "  " << T << "* const vals = b" << f.val << ";\n"
        // 8-aligned body: 8 keys in one 16-byte load, 8 values in two
        // 16-byte stores; the unaligned head and tail one by one
        << "  const int up8 = (lo + 7) & ~7, dn8 = hi & ~7;\n"
        << "  const int lo8 = up8 < hi ? up8 : hi;\n"
        << "  const int hi8 = dn8 > lo8 ? dn8 : lo8;\n"
        << "  for (int j = lo + (int)threadIdx.x; j < lo8; j += " << GT << ") vals[j] = tab[keys[j]];\n"
        << "  for (int j = hi8 + (int)threadIdx.x; j < hi; j += " << GT << ") vals[j] = tab[keys[j]];\n"
        << "  for (int j0 = lo8 + 8 * (int)threadIdx.x; j0 < hi8; j0 += " << 32 * GT << ") {\n"
        << "    u16x8 kv[4];\n"
        << "#pragma unroll\n"
        << "    for (int u = 0; u < 4; u++) kv[u] = *(const u16x8*)(keys + (j0 + u * " << 8 * GT << " < hi8 ? j0 + u * "
        << 8 * GT << " : j0));\n"
        << "#pragma unroll\n"
        << "    for (int u = 0; u < 4; u++)\n"
        << "      if (j0 + u * " << 8 * GT << " < hi8) {\n"
        << "        const v4 a = {tab[kv[u][0]], tab[kv[u][1]], tab[kv[u][2]], tab[kv[u][3]]};\n"
        << "        const v4 c = {tab[kv[u][4]], tab[kv[u][5]], tab[kv[u][6]], tab[kv[u][7]]};\n"
        << "        *(v4*)(vals + j0 + u * " << 8 * GT << ") = a;\n"
        << "        *(v4*)(vals + j0 + u * " << 8 * GT << " + 4) = c;\n"
        << "      }\n"
        << "  }\n"
        << "}\n";
      }
      src << k.str();
      std::vector<int> sargs = {lead, f.key, gb.h, f.val};
      if (f.windows) sargs.push_back(f.wtab);
      ks.push_back(add_kernel(kname + "_slices", sargs, (int)(gb.P * Wg), (int)GT, "gather_slices"));
    }
    auto unpartition = [&](const std::string &sfx, const PassOut &o, int from, int to, bool flag) {
      std::vector<int> args = {o.meta, o.slot, from, to};
      std::ostringstream k;
      k << "extern \"C\" __global__ __launch_bounds__(" << GT << ") void " << kname << "_unpartition" << sfx
        << "(const int* __restrict__ b" << o.meta << ", const int* __restrict__ b" << o.slot << ", const " << T
        << "* __restrict__ b" << from << ", " << T << "* __restrict__ b" << to;
      if (o.nbuf >= 0) {
        k << ", const int* __restrict__ b" << o.nbuf;
        args.push_back(o.nbuf);
      }
      if (o.windows) {
        k << ", const int* __restrict__ b" << o.wstart << ", const int* __restrict__ b" << o.wtab;
        args.push_back(o.wstart);
        args.push_back(o.wtab);
      }
      if (flag) {
        k << ", int* __restrict__ err";
        args.push_back(err_buf());
      }
      const int64_t KM = o.kmax();
      const int64_t E = o.TILE / GT, VB = cdiv(o.TILE, 8 * GT);  // slots, 8-element groups per thread
      // Streaming: 1 the output's stores, 2 the slot and region loads. The
      // tile-local unpartition streams both (config 3: 139 -> 121 us, and
      // the next step's partition 201 -> 191, its lines no longer dirty in
      // the MALL); the two-level passes keep plain accesses (3b's last
      // unpartition 146 -> 156 us streamed). gb_nt sets it.
      const int64_t gbnt = tune("gb_nt", o.local && !o.windows ? 3 : 0);
      const std::string zero = zero_of(n.dt);
      if (o.windows) {
        // a window's region, read whole into LDS; each element of the
        // window (contiguous in the coarse order, at any alignment) takes
        // the value at its slot. Every element of a window has a slot.
        const int64_t VR = cdiv(o.RS, 8 * GT);
        k << ") {\n"
          << "  typedef " << v4 << " v4;\n"
          << "  __shared__ __align__(16) " << T << " st[" << o.RS << "];\n"
          << "  const int ft = blockIdx.x;\n"
          << window_at(o, "ft")
          << "  const unsigned short* const sl = (const unsigned short*)b" << o.slot << ";\n"
          << "  unsigned sv[" << E << "];\n"
          << "#pragma unroll\n"
          << "  for (int u = 0; u < " << E << "; u++) {\n"
          << "    const int i = (int)threadIdx.x + u * " << GT << ";\n"
          << "    sv[u] = i < wn_ ? sl[wb_ + i] : 0u;\n"
          << "  }\n"
          << "  const int tot = ((const int2*)b" << o.meta << ")[(size_t)" << 64 * o.NTT << " + ft].x;\n"
          << "  const " << T << "* const rg = b" << from << " + (size_t)ft * " << o.RS << ";\n"
          << "  v4 ra[" << VR << "], rc[" << VR << "];\n"
          << "#pragma unroll\n"
          << "  for (int u = 0; u < " << VR << "; u++) {\n"
          << "    const int s = 8 * ((int)threadIdx.x + " << GT << " * u);\n"
          << ((gbnt & 2) ? "    if (s < tot) { ra[u] = __builtin_nontemporal_load((const v4*)(rg + s)); "
                                       "rc[u] = __builtin_nontemporal_load((const v4*)(rg + s + 4)); }\n"
                                     : "    if (s < tot) { ra[u] = *(const v4*)(rg + s); rc[u] = *(const v4*)(rg + s + 4); }\n")
          << "  }\n"
          << "#pragma unroll\n"
          << "  for (int u = 0; u < " << VR << "; u++) {\n"
          << "    const int s = 8 * ((int)threadIdx.x + " << GT << " * u);\n"
          << "    if (s < tot) { *(v4*)(st + s) = ra[u]; *(v4*)(st + s + 4) = rc[u]; }\n"
          << "  }\n"
          << "  __syncthreads();\n"
          << "#pragma unroll\n"
          << "  for (int u = 0; u < " << E << "; u++) {\n"
          << "    const int i = (int)threadIdx.x + u * " << GT << ";\n"
          << "    if (i < wn_) b" << to << "[wb_ + i] = st[sv[u]];\n"
          << "  }\n"
          << "}\n";
        src << k.str();
        ks.push_back(add_kernel(kname + "_unpartition" + sfx, args, (int)o.NTT, (int)GT, "gather_unpartition"));
        return;
      }
      if (o.local) {
        // the tile's region, read whole into LDS, then every element takes
        // the value at its slot
        const int64_t VR = cdiv(o.RS, 8 * GT);  // 8-element groups of the region per thread
        k << ") {\n"
          << "  typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));\n"
          << "  typedef " << v4 << " v4;\n"
          << "  __shared__ __align__(16) " << T << " st[" << o.RS << "];\n"
          << "  const int g = blockIdx.x / " << o.TPC << ", kt = blockIdx.x - g * " << o.TPC << ";\n"
          << "  const int nv_ = " << o.nvalid << ";\n"
          << "  const int lo = g * " << o.C << ";\n"
          << "  const int hc = lo + " << o.C << " < nv_ ? lo + " << o.C << " : nv_;\n"
          << "  const int t0 = lo + kt * " << o.TILE << ";\n"
          << "  if (t0 >= hc) return;  // a tile the partition never had: the whole workgroup leaves\n"
          << "  const int hi = t0 + " << o.TILE << " < hc ? t0 + " << o.TILE << " : hc;\n"
          << "  const unsigned short* const sl = (const unsigned short*)b" << o.slot << ";\n"
          << "  " << T << "* const dst = b" << to << ";\n"
          << "  u16x8 sv[" << VB << "];\n"
          << "#pragma unroll\n"
          << "  for (int u = 0; u < " << VB << "; u++) {\n"
          << "    const int i = t0 + 8 * ((int)threadIdx.x + " << GT << " * u);\n"
          << ((gbnt & 2) ? "    if (i + 8 <= hi) sv[u] = __builtin_nontemporal_load((const u16x8*)(sl + i));\n"
                                       : "    if (i + 8 <= hi) sv[u] = *(const u16x8*)(sl + i);\n")
          << "    else sv[u] = (u16x8)(unsigned short)0xffffu;\n"
          << "  }\n"
          << "  const int tot = ((const int2*)b" << o.meta << ")[(size_t)" << o.PB * o.NTT << " + blockIdx.x].x;\n"
          << "  const " << T << "* const rg = b" << from << " + (size_t)blockIdx.x * " << o.RS << ";\n"
          << "  v4 ra[" << VR << "], rc[" << VR << "];\n"
          << "#pragma unroll\n"
          << "  for (int u = 0; u < " << VR << "; u++) {\n"
          << "    const int s = 8 * ((int)threadIdx.x + " << GT << " * u);\n"
          << ((gbnt & 2) ? "    if (s < tot) { ra[u] = __builtin_nontemporal_load((const v4*)(rg + s)); "
                                       "rc[u] = __builtin_nontemporal_load((const v4*)(rg + s + 4)); }\n"
                                     : "    if (s < tot) { ra[u] = *(const v4*)(rg + s); rc[u] = *(const v4*)(rg + s + 4); }\n")
          << "  }\n"
          << "#pragma unroll\n"
          << "  for (int u = 0; u < " << VR << "; u++) {\n"
          << "    const int s = 8 * ((int)threadIdx.x + " << GT << " * u);\n"
          << "    if (s < tot) { *(v4*)(st + s) = ra[u]; *(v4*)(st + s + 4) = rc[u]; }\n"
          << "  }\n"
          << "  __syncthreads();\n";
      } else {
      k << ") {\n"
        << "  typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));\n"
        << "  typedef " << v4 << " v4;\n"
        << "  __shared__ int mt[" << KM + 1 << "];\n"
        << "  __shared__ int mc[" << KM << "];\n"
        << "  __shared__ " << T << " st[" << o.TILE << "];\n"
        << "  const int g = blockIdx.x / " << o.TPC << ", kt = blockIdx.x - g * " << o.TPC << ";\n"
        << "  const int nv_ = " << o.nvalid << ";\n"
        << "  const int lo = g * " << o.C << ";\n"
        << "  const int hc = lo + " << o.C << " < nv_ ? lo + " << o.C << " : nv_;\n"
        << "  const int t0 = lo + kt * " << o.TILE << ";\n"
        << "  if (t0 >= hc) return;  // a tile the partition never had: the whole workgroup leaves\n"
        << "  const int hi = t0 + " << o.TILE << " < hc ? t0 + " << o.TILE << " : hc;\n"
        << "  const int* const meta = b" << o.meta << " + (size_t)blockIdx.x * " << o.meta_stride() << ";\n"
        << "  const unsigned short* const sl = (const unsigned short*)b" << o.slot << ";\n"
        << "  " << T << "* const dst = b" << to << ";\n"
        // this thread's element slots, 8 per group in one 16-byte load (t0 is
        // a multiple of 256), requested before anything else; a group that
        // runs past hi is read one by one later
        << "  u16x8 sv[" << VB << "];\n"
        << "#pragma unroll\n"
        << "  for (int u = 0; u < " << VB << "; u++) {\n"
        << "    const int i = t0 + 8 * ((int)threadIdx.x + " << GT << " * u);\n"
        << "    if (i + 8 <= hi) sv[u] = *(const u16x8*)(sl + i);\n"
        << "    else sv[u] = (u16x8)(unsigned short)0xffffu;\n"
        << "  }\n"
        << "  const int nk = meta[0];\n"
        << "  for (int c = threadIdx.x; c <= nk; c += " << GT << ") mt[c] = meta[1 + c];\n"
        << "  for (int c = threadIdx.x; c < nk; c += " << GT << ") mc[c] = meta[" << KM + 2 << " + c];\n"
        << "  __syncthreads();\n"
        << "  const int tot = mt[nk];\n"
        // the tile's runs into LDS in its bucket-grouped order: slot s lies in
        // the last non-empty bucket whose tile-local start is <= s; all of a
        // thread's slots searched, then all their loads issued together
        << "  if (tot > 0) {\n"
        // Each wave takes a contiguous quarter of the slots, 64 at a time;
        // a lane's bucket is the last one starting at or before its slot:
        // one search for the wave's first slot (the same for every lane),
        // then each lane probes forward from where lane 63 stopped the
        // previous time (runs are about as long as a wave, so one or two
        // probes). All addresses first, then all loads together.
        << "    const int lane = threadIdx.x & 63;\n"
        << "    const int sw = (int)(threadIdx.x >> 6) * " << E * 64 << ";\n"
        << "    int aw = 0;\n"
        << "    for (int step = nk > 1 ? 1 << (31 - __clz(nk - 1)) : 0; step >= 1; step >>= 1) {\n"
        << "      const int m = aw + step;\n"
        << "      if (m < nk && mt[m] <= sw) aw = m;\n"
        << "    }\n"
        << "    int at[" << E << "];\n"
        << "#pragma unroll\n"
        << "    for (int u = 0; u < " << E << "; u++) {\n"
        << "      const int s = sw + u * 64 + lane;\n"
        << "      int a = aw;\n"
        << "      while (a + 1 < nk && mt[a + 1] <= s) a++;\n"
        << "      at[u] = s < tot ? mc[a] + (s - mt[a]) : mc[0];\n"
        << "      aw = __shfl(a, 63);\n"
        << "    }\n"
        << "    " << T << " v[" << E << "];\n"
        << "#pragma unroll\n"
        << "    for (int u = 0; u < " << E << "; u++) v[u] = b" << from << "[at[u]];\n"
        << "#pragma unroll\n"
        << "    for (int u = 0; u < " << E << "; u++)\n"
        << "      if (sw + u * 64 + lane < tot) st[sw + u * 64 + lane] = v[u];\n"
        << "  }\n"
        << "  __syncthreads();\n";
      }
      k << "  bool bad = false;\n"
        << "#pragma unroll\n"
        << "  for (int u = 0; u < " << VB << "; u++) {\n"
        << "    const int i = t0 + 8 * ((int)threadIdx.x + " << GT << " * u);\n"
        << "    if (i + 8 <= hi) {\n"
        << "      " << T << " x[8];\n"
        << "#pragma unroll\n"
        << "      for (int e = 0; e < 8; e++) {\n"
        << "        const unsigned v = sv[u][e];\n"
        << "        x[e] = v != 0xffffu ? st[v] : " << zero << ";\n"
        << "        bad = bad || v == 0xffffu;\n"
        << "      }\n"
        << "      const v4 a = {x[0], x[1], x[2], x[3]}, c = {x[4], x[5], x[6], x[7]};\n"
        << ((gbnt & 1) ? "      __builtin_nontemporal_store(a, (v4*)(dst + i));\n"
                                     "      __builtin_nontemporal_store(c, (v4*)(dst + i + 4));\n"
                                   : "      *(v4*)(dst + i) = a;\n"
                                     "      *(v4*)(dst + i + 4) = c;\n")
        << "    } else {\n"
        << "      for (int e = i; e < hi; e++) {\n"
        << "        const unsigned v = sl[e];\n"
        << "        dst[e] = v != 0xffffu ? st[v] : " << zero << ";\n"
        << "        bad = bad || v == 0xffffu;\n"
        << "      }\n"
        << "    }\n"
        << "  }\n";
      if (flag) k << "  if (bad) cc_flag(err, 1);\n";
      k << "}\n";
      src << k.str();
      ks.push_back(add_kernel(kname + "_unpartition" + sfx, args, (int)(o.G * o.TPC), (int)GT, "gather_unpartition"));
    };
    if (gb.coarse.slot >= 0) {
      unpartition("2", f, f.val, gb.coarse.val, false);
      unpartition("", gb.coarse, gb.coarse.val, out, true);
    } else {
      unpartition("", f, f.val, out, true);
    }
    for (const PassOut *o : {&gb.fin, &gb.coarse})
      for (int b : {o->start, o->key, o->val, o->slot, o->meta, o->nbuf, o->wtab})
        if (b >= 0) free_after[b] = r;
    return ks;
  }

  // Block tile edge of the matrix-core kernels (square tiles; four waves of
  // BM/2 x BM/2).
  static int64_t mfma_bm(DT dt) {
    if (dt == DT::F64) return tune("mm_f64_bm", 64) == 128 ? 128 : 64;
    return 128;
  }
  // k-tile depth: 16, or 32 where K allows it and the knob asks for it.
  static int64_t mfma_bk(DT dt, int64_t K) {
    int64_t want = tune(dt == DT::F64 ? "mm_f64_bk" : "mm_bk", 16);
    return want == 32 && K % 32 == 0 ? 32 : 16;
  }

  // ---- Matmul on the matrix cores ------------------------------------------
  // f32: v_mfma_f32_32x32x2f32, block tile 128x128x16, four waves of 64x64.
  // f64: v_mfma_f64_16x16x4f64, block tile 64x64x16, four waves of 32x32.
  // Within a 16-deep k tile, lane group g (of 64/MT groups) takes the k
  // values g*S .. g*S+S-1 in order (A and B use the same permutation), so a
  // lane's operands for the whole tile are one contiguous run along k.
  // Each operand is staged in the LDS layout that matches its source:
  // k-contiguous rows for A and for a transposed B, MN-contiguous rows for B
  // and for a transposed A, so global loads stay coalesced either way;
  // operands that are fused expressions are computed into the k-contiguous
  // layout. Two LDS buffers, next tile prefetched into registers. Products
  // accumulate on the matrix cores, so f32 sums are not in the
  // interpreter's order: results match it to rounding, not bit for bit.
  std::vector<int> lower_matmul_mfma(int t, int64_t M, int64_t N, int64_t K) {
    const TNode &n = g.ts[t];
    std::string id = std::to_string(n.id);
    std::string kname = "k_" + id;
    bool f64 = n.dt == DT::F64;
    std::string T = dt_ctype(n.dt);
    int out = buf_of[t];
    const int64_t BM = mfma_bm(n.dt), BK = mfma_bk(n.dt, K), MT = f64 ? 16 : 32;
    const int64_t G = 64 / MT;    // lane groups along k
    const int64_t S = BK / G;     // k steps per tile held by one lane
    const int64_t WT = BM / 2;    // wave tile
    const int64_t RT = WT / MT;   // instruction tiles per wave side
    const int64_t VEC = 16 / dt_size(n.dt);        // elements per 16-byte access
    const int64_t PER = BM * BK / 256;             // elements per thread per operand tile
    // row strides padded by whole 16-byte vectors (alignment kept); the pads
    // spread rows over LDS banks
    const int64_t KP = BK + VEC * std::max<int64_t>(0, tune("mm_kpad", 1));  // k-contiguous row stride
    const int64_t MP = BM + VEC * std::max<int64_t>(0, tune("mm_mpad", 1));  // mn-contiguous row stride
    // Operand modes: 0 direct buffer, 1 transpose of a buffer, 2 fused expression.
    struct Opnd {
      int mode;
      int buf;
      bool kcontig;
      ElemFn fn;
    };
    auto classify = [&](int op, bool is_a) {
      Opnd o;
      o.buf = -1;
      if (plan.materialized[op]) {
        o.mode = 0;
        o.buf = buf_of[op];
        o.kcontig = is_a;  // A[m][k] rows are k-contiguous; B[k][n] rows are n-contiguous
      } else if (transpose_source(g, op) >= 0 && plan.materialized[transpose_source(g, op)] &&
                 !plan.materialized[g.ts[op].a]) {
        o.mode = 1;
        o.buf = buf_of[transpose_source(g, op)];
        o.kcontig = !is_a;
      } else {
        o.mode = 2;
        o.kcontig = true;
        o.fn = gen.element_fn(std::string(is_a ? "fa_" : "fb_") + id, op, false, false);
        src << o.fn.code;
      }
      return o;
    };
    Opnd A = classify(n.a, true), B = classify(n.b, false);
    Params p;
    for (Opnd *o : {&A, &B}) {
      if (o->mode == 2) add_in(p, o->fn);
      else {
        bool dup = false;
        for (int x : p.in) dup |= x == o->buf;
        if (!dup) p.in.push_back(o->buf);
      }
    }
    p.out.push_back(out);
    std::vector<int> args;
    std::string params = param_list(p, args);
    const int64_t ALDS = A.kcontig ? BM * KP : BK * MP;
    const int64_t BLDS = B.kcontig ? BM * KP : BK * MP;
    std::string V = f64 ? "cc_v2<double>" : "cc_v4<float>";  // one 16-byte access
    // The prefetch registers are native vectors: staged through arrays of
    // a struct type, the global load and its later LDS store were turned
    // into one global-to-LDS copy at the store, after the matrix-core
    // work, so the next tile's loads were not in flight during it.
    const std::string RV = f64 ? "cc_d2v" : "cc_f4v";
    const int64_t NR = PER / VEC;
    std::ostringstream k;
    // Global -> registers for one operand tile. `base` is the tile's first
    // row (m for A, n for B) along MN; kt the tile's first k.
    auto gload = [&](const Opnd &o, bool is_a, const std::string &reg) {
      std::ostringstream l;
      std::string mnb = is_a ? "bm" : "bn";
      int64_t MNtot = is_a ? M : N;
      if (o.kcontig) {
        // thread -> (row r, k offset kk) with PER consecutive k
        l << "    { const int r = threadIdx.x / " << BK / PER << ", kk = (threadIdx.x % " << BK / PER << ") * " << PER
          << ";\n";
        if (o.mode == 2) {
          for (int64_t c = 0; c < PER; c++) {
            std::string idx = is_a ? "(" + mnb + " + r) * " + std::to_string(K) + " + kt + kk + " + std::to_string(c)
                                   : "(kt + kk + " + std::to_string(c) + ") * " + std::to_string(N) + " + " + mnb +
                                         " + r";
            l << "      " << reg << "[" << c / VEC << "][" << c % VEC << "] = " << o.fn.call_scalar(idx) << ";\n";
          }
        } else {
          // direct A ([M][K]) or transposed B (source [N][K]): row length K
          l << "      const " << T << "* s = b" << o.buf << " + (size_t)(" << mnb << " + r) * " << K << " + kt + kk;\n";
          for (int64_t c = 0; c < PER; c += VEC)
            l << "      " << reg << "[" << c / VEC << "] = *(const " << RV << "*)(s + " << c << ");\n";
        }
        l << "    }\n";
      } else {
        // thread -> (k row kk, MN offset c0) with PER consecutive MN
        l << "    { const int kk = threadIdx.x / " << BM / PER << ", c0 = (threadIdx.x % " << BM / PER << ") * " << PER
          << ";\n"
          << "      const " << T << "* s = b" << o.buf << " + (size_t)(kt + kk) * " << MNtot << " + " << mnb
          << " + c0;\n";
        for (int64_t c = 0; c < PER; c += VEC)
          l << "      " << reg << "[" << c / VEC << "] = *(const " << RV << "*)(s + " << c << ");\n";
        l << "    }\n";
      }
      return l.str();
    };
    auto lstore = [&](const Opnd &o, const std::string &lds, const std::string &reg) {
      std::ostringstream l;
      if (o.kcontig)
        l << "    { const int r = threadIdx.x / " << BK / PER << ", kk = (threadIdx.x % " << BK / PER << ") * " << PER
          << ";\n"
          << "      " << T << "* d = " << lds << " + r * " << KP << " + kk;\n";
      else
        l << "    { const int kk = threadIdx.x / " << BM / PER << ", c0 = (threadIdx.x % " << BM / PER << ") * "
          << PER << ";\n"
          << "      " << T << "* d = " << lds << " + kk * " << MP << " + c0;\n";
      for (int64_t c = 0; c < PER; c += VEC)
        l << "      *(" << RV << "*)(d + " << c << ") = " << reg << "[" << c / VEC << "];\n";
      l << "    }\n";
      return l.str();
    };
    // LDS -> fragment registers: lane's S consecutive k for instruction tile rt
    auto fragload = [&](const Opnd &o, const std::string &lds, const std::string &frag, const std::string &mn0) {
      std::ostringstream l;
      l << "#pragma unroll\n"
        << "      for (int rt = 0; rt < " << RT << "; rt++) {\n"
        << "        const int mn = " << mn0 << " + rt * " << MT << " + (lane % " << MT << ");\n"
        << "        const int k0 = (lane / " << MT << ") * " << S << ";\n";
      if (o.kcontig) {
        for (int64_t c = 0; c < S; c += VEC)
          l << "        *(" << V << "*)&" << frag << "[rt][" << c << "] = *(const " << V << "*)(" << lds << " + mn * "
            << KP << " + k0 + " << c << ");\n";
      } else {
        l << "#pragma unroll\n"
          << "        for (int s2 = 0; s2 < " << S << "; s2++) " << frag << "[rt][s2] = " << lds << "[(k0 + s2) * " << MP
          << " + mn];\n";
      }
      l << "      }\n";
      return l.str();
    };
    std::string accT = f64 ? "cc_f64x4" : "cc_f32x16";
    int64_t NACC = f64 ? 4 : 16;
    std::string mfma = f64 ? "__builtin_amdgcn_mfma_f64_16x16x4f64" : "__builtin_amdgcn_mfma_f32_32x32x2f32";
    int64_t tiles_m = M / BM, tiles_n = N / BM, ntiles = tiles_m * tiles_n;
    // f64: one LDS buffer, refilled between two barriers (the fragments are
    // in registers by the first), and a four-waves-a-SIMD register budget,
    // which also keeps the accumulators in ordinary vector registers: at
    // 2048^3, 47 -> 52 TFLOP/s against the double-buffered kernel
    // (mm_f64_single=0, mm_f64_waves=0 restore it). f32 measured no gain
    // from either.
    const bool single = f64 && tune("mm_f64_single", 1) != 0;
    const int64_t waves = f64 ? std::max<int64_t>(0, std::min<int64_t>(8, tune("mm_f64_waves", 4))) : 0;
    k << "typedef " << T << " " << accT << " __attribute__((ext_vector_type(" << NACC << ")));\n"
      << "extern \"C\" __global__ __launch_bounds__(256) ";
    if (waves > 0) k << "__attribute__((amdgpu_waves_per_eu(" << waves << ", " << waves << "))) ";
    k << "void " << kname << "(" << params << ") {\n"
      << "  __shared__ __attribute__((aligned(16))) " << T << " As[" << (single ? 1 : 2) << "][" << ALDS << "];\n"
      << "  __shared__ __attribute__((aligned(16))) " << T << " Bs[" << (single ? 1 : 2) << "][" << BLDS << "];\n"
      << "  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;\n"
      << "  const int wm = (wid >> 1) * " << WT << ", wn = (wid & 1) * " << WT << ";\n"
      // blocks are dispatched round-robin over the 8 XCDs; give each XCD a
      // contiguous run of tiles so its L2 sees shared A row panels.
      << "  int tile = blockIdx.x;\n";
    if (ntiles % 8 == 0) {
      const int64_t TX = ntiles / 8, RX = TX % tiles_n == 0 ? TX / tiles_n : 0;
      k << "  tile = (tile % 8) * " << TX << " + tile / 8;\n";
      // Within an XCD's RX whole tile rows, walk column by column, so the
      // tiles resident together span RX row panels of A and few column
      // panels of B instead of one row panel and every column panel.
      if (RX > 1 && tune("mm_xcd_cols", 1))
        k << "  { const int x = tile / " << TX << ", l = tile - x * " << TX << "; tile = x * " << TX << " + (l % " << RX
          << ") * " << tiles_n << " + l / " << RX << "; }\n";
    }
    k << "  const int bm = (tile / " << tiles_n << ") * " << BM << ", bn = (tile % " << tiles_n << ") * " << BM << ";\n"
      << "  " << accT << " acc[" << RT << "][" << RT << "];\n"
      << "#pragma unroll\n"
      << "  for (int i = 0; i < " << RT << "; i++)\n"
      << "#pragma unroll\n"
      << "    for (int j = 0; j < " << RT << "; j++) acc[i][j] = (" << accT << ")(0);\n"
      << "  " << RV << " ra[" << NR << "], rb[" << NR << "];\n";
    // Two-level accumulation (f32): the matrix cores sum KC-deep chunks into
    // `acc`, which is folded into `tot` with plain adds and cleared. Error
    // then grows with sqrt(KC) + sqrt(K / KC) instead of sqrt(K): for N(0,1)
    // operands at K = 4096 and KC = 256 about 3e-5 of (1 + |exact|), against
    // about 1.7e-4 for one f32 accumulator (and for the interpreter's own
    // sequential sum). KC = mm_chunk_k, 256 by default.
    int64_t KCT = f64 ? 0 : std::max<int64_t>(0, tune("mm_chunk_k", 256) / BK);
    if (KCT > 0 && (K / BK) % KCT != 0) KCT = 0;
    if (KCT > 0)
      k << "  " << accT << " tot[" << RT << "][" << RT << "];\n"
        << "#pragma unroll\n"
        << "  for (int i = 0; i < " << RT << "; i++)\n"
        << "#pragma unroll\n"
        << "    for (int j = 0; j < " << RT << "; j++) tot[i][j] = (" << accT << ")(0);\n";
    k << "  int kt = 0;\n"
      << gload(A, true, "ra") << gload(B, false, "rb") << lstore(A, "As[0]", "ra") << lstore(B, "Bs[0]", "rb")
      << "  __syncthreads();\n"
      << "  for (int it = 0; it < " << K / BK << "; it++) {\n"
      << "    const int buf = " << (single ? "0" : "it & 1") << ";\n"
      << "    kt = (it + 1) * " << BK << ";\n"
      << "    if (it + 1 < " << K / BK << ") {\n"
      << gload(A, true, "ra") << gload(B, false, "rb") << "    }\n"
      // keeps the scheduler from sinking the next tile's loads to their
      // LDS stores (to save registers), which left them unhidden
      << "    __builtin_amdgcn_sched_barrier(0);\n"
      << "    {\n"
      << "      __attribute__((aligned(16))) " << T << " fa[" << RT << "][" << S << "], fb[" << RT << "][" << S << "];\n"
      << "      const " << T << "* const al = As[buf];\n"
      << "      const " << T << "* const bl = Bs[buf];\n"
      << fragload(A, "al", "fa", "wm") << fragload(B, "bl", "fb", "wn");
    if (single)  // every wave holds its fragments: the buffer takes the next tile
      k << "      __syncthreads();\n"
        << "      if (it + 1 < " << K / BK << ") {\n"
        << lstore(A, "As[0]", "ra") << lstore(B, "Bs[0]", "rb") << "      }\n";
    k << "#pragma unroll\n"
      << "      for (int s2 = 0; s2 < " << S << "; s2++)\n"
      << "#pragma unroll\n"
      << "        for (int i = 0; i < " << RT << "; i++)\n"
      << "#pragma unroll\n"
      << "          for (int j = 0; j < " << RT << "; j++) acc[i][j] = " << mfma
      << "(fa[i][s2], fb[j][s2], acc[i][j], 0, 0, 0);\n"
      << "    }\n";
    if (!single)
      k << "    if (it + 1 < " << K / BK << ") {\n"
        << lstore(A, "As[buf ^ 1]", "ra") << lstore(B, "Bs[buf ^ 1]", "rb") << "    }\n";
    if (KCT > 0)
      k << "    if ((it + 1) % " << KCT << " == 0) {\n"
        << "#pragma unroll\n"
        << "      for (int i = 0; i < " << RT << "; i++)\n"
        << "#pragma unroll\n"
        << "        for (int j = 0; j < " << RT << "; j++) { tot[i][j] += acc[i][j]; acc[i][j] = (" << accT << ")(0); }\n"
        << "    }\n";
    k << "    __syncthreads();\n"
      << "  }\n"
      // epilogue: the accumulator layout of the instruction
      << "#pragma unroll\n"
      << "  for (int i = 0; i < " << RT << "; i++)\n"
      << "#pragma unroll\n"
      << "    for (int j = 0; j < " << RT << "; j++) {\n"
      << "      const int col = bn + wn + j * " << MT << " + (lane % " << MT << ");\n"
      << "#pragma unroll\n"
      << "      for (int r = 0; r < " << NACC << "; r++) {\n";
    if (f64)  // the f64 instruction interleaves rows: lane group g holds rows g, g+4, g+8, g+12
      k << "        const int row = bm + wm + i * 16 + (lane / 16) + 4 * r;\n";
    else
      k << "        const int row = bm + wm + i * 32 + (r / 4) * 8 + (lane / 32) * 4 + (r % 4);\n";
    k << "        b" << out << "[(size_t)row * " << N << " + col] = " << (KCT > 0 ? "tot" : "acc") << "[i][j][r];\n"
      << "      }\n"
      << "    }\n"
      << "}\n";
    src << k.str();
    std::string role = std::string("matmul_mfma_") + (f64 ? "f64" : "f32") + "_" + "a" + std::to_string(A.mode) +
                       "b" + std::to_string(B.mode);
    return {add_kernel(kname, args, (int)ntiles, 256, role)};
  }

  // ---- Skinny matmul: split over k ------------------------------------------
  // For products with few outputs and a long k (LSM's X^T X : [3;n] x [n;3],
  // n = 65536) the 16x16 tiling launches one workgroup that walks all of k.
  // Here workgroup g folds the k-chunk [g*KC, (g+1)*KC): thread t takes
  // k = k0 + t, k0 + t + 256, ... for every output, the partial sums are
  // reduced across the workgroup, and a second kernel adds the G partials
  // of each output in g order. Products and sums are rounded separately
  // (no FMA), as the interpreter does (R9); the summation order differs
  // from its k-ascending one, so float results match to rounding.
  std::vector<int> lower_matmul_splitk(int t, int64_t M, int64_t N, int64_t K, const ElemFn &fa, const ElemFn &fb) {
    const TNode &n = g.ts[t];
    std::string id = std::to_string(n.id);
    std::string kname = "k_" + id;
    std::string T = dt_ctype(n.dt);
    std::string acc = n.dt == DT::I32 ? "cc_u32" : (n.dt == DT::I64 ? "cc_u64" : T);  // integers wrap
    int out = buf_of[t];
    const int64_t MN = M * N;
    int64_t G = std::max<int64_t>(1, std::min<int64_t>(tune("mm_splitk_groups", 256), cdiv(K, 512)));
    int64_t KC = cdiv(cdiv(K, G), 256) * 256;
    G = cdiv(K, KC);
    int part = add_buf("t" + id + "_kpart", n.dt, G * MN, BufRole::Scratch);
    Params p;
    add_in(p, fa);
    add_in(p, fb);
    p.out.push_back(part);
    std::vector<int> args;
    std::string params = param_list(p, args);
    std::ostringstream k;
    k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "_splitk(" << params << ") {\n"
      << "  __shared__ " << acc << " wpart[4][" << MN << "];\n"
      << "  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;\n"
      << "  " << acc << " s[" << MN << "];\n"
      << "#pragma unroll\n"
      << "  for (int q = 0; q < " << MN << "; q++) s[q] = (" << acc << ")0;\n"
      << "  const int k0 = blockIdx.x * " << KC << ";\n"
      << "  const int k1 = k0 + " << KC << " < " << K << " ? k0 + " << KC << " : " << K << ";\n"
      << "  for (int kk = k0 + (int)threadIdx.x; kk < k1; kk += 256) {\n"
      << "    " << T << " a[" << M << "], b[" << N << "];\n";
    for (int64_t m = 0; m < M; m++)
      k << "    a[" << m << "] = " << fa.call_scalar(std::to_string(m * K) + " + kk") << ";\n";
    for (int64_t c = 0; c < N; c++)
      k << "    b[" << c << "] = " << fb.call_scalar("kk * " + std::to_string(N) + " + " + std::to_string(c)) << ";\n";
    k << "#pragma unroll\n"
      << "    for (int m = 0; m < " << M << "; m++)\n"
      << "#pragma unroll\n"
      << "      for (int c = 0; c < " << N << "; c++) {\n";
    if (n.dt == DT::I32 || n.dt == DT::I64)
      k << "        s[m * " << N << " + c] += (" << acc << ")a[m] * (" << acc << ")b[c];\n";
    else
      k << "        const " << T << " pr = a[m] * b[c];\n"
        << "        s[m * " << N << " + c] = s[m * " << N << " + c] + pr;\n";
    k << "      }\n"
      << "  }\n"
      << "#pragma unroll\n"
      << "  for (int q = 0; q < " << MN << "; q++) {\n"
      << "    " << acc << " v = s[q];\n"
      << "    for (int off = 32; off > 0; off >>= 1) v = v + __shfl_xor(v, off);\n"
      << "    if (lane == 0) wpart[wid][q] = v;\n"
      << "  }\n"
      << "  __syncthreads();\n"
      << "  for (int q = threadIdx.x; q < " << MN << "; q += 256)\n"
      << "    b" << part << "[(size_t)blockIdx.x * " << MN << " + q] = (" << T << ")(((wpart[0][q] + wpart[1][q]) + wpart[2][q]) + wpart[3][q]);\n"
      << "}\n";
    k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "_ksum(const " << T << "* __restrict__ b"
      << part << ", " << T << "* __restrict__ b" << out << ") {\n"
      << "  for (int q = blockIdx.x * 256 + threadIdx.x; q < " << MN << "; q += gridDim.x * 256) {\n"
      << "    " << acc << " v = (" << acc << ")b" << part << "[q];\n"
      << "    for (int gg = 1; gg < " << G << "; gg++) v = v + (" << acc << ")b" << part << "[(size_t)gg * " << MN
      << " + q];\n"
      << "    b" << out << "[q] = (" << T << ")v;\n"
      << "  }\n"
      << "}\n";
    src << k.str();
    int k1 = add_kernel(kname + "_splitk", args, (int)G, 256, "matmul_splitk");
    int k2 = add_kernel(kname + "_ksum", {part, out}, (int)std::max<int64_t>(1, cdiv(MN, 256)), 256, "matmul_ksum");
    return {k1, k2};
  }

  // ---- Matmul root (K11) --------------------------------------------------
  // Generic tiled product: one output per thread, k ascending, each product
  // and sum rounded separately, zero-padded edge tiles. For float dtypes
  // this reproduces the interpreter's rounding exactly (R9).
  std::vector<int> lower_matmul(int t) {
    const TNode &n = g.ts[t];
    std::string id = std::to_string(n.id);
    std::string kname = "k_" + id;
    std::string T = dt_ctype(n.dt);
    int out = buf_of[t];
    int64_t M = n.shape[0], N = n.shape[1];
    int64_t K = g.ts[n.a].shape[1];
    if (M == 0 || N == 0) return {};
    if (dt_is_float(n.dt) && K > 0 && tune("mm_mfma", 1)) {
      int64_t BM = mfma_bm(n.dt);
      if (M % BM == 0 && N % BM == 0 && K % mfma_bk(n.dt, K) == 0) return lower_matmul_mfma(t, M, N, K);
    }
    ElemFn fa = gen.element_fn("fa_" + id, n.a, false, false);
    ElemFn fb = gen.element_fn("fb_" + id, n.b, false, false);
    src << fa.code << fb.code;
    if (K > 0 && M * N <= tune("mm_splitk_outputs", 32) && cdiv(M, 16) * cdiv(N, 16) < 64 &&
        K >= tune("mm_splitk_min_k", 4096))
      return lower_matmul_splitk(t, M, N, K, fa, fb);
    Params p;
    add_in(p, fa);
    add_in(p, fb);
    p.out.push_back(out);
    std::vector<int> args;
    std::string params = param_list(p, args);
    auto mul = [&](const std::string &a, const std::string &b) {
      if (dt_is_float(n.dt)) return "(" + a + " * " + b + ")";
      std::string U = n.dt == DT::I64 ? "cc_u64" : "cc_u32";
      return "((" + T + ")((" + U + ")(" + a + ") * (" + U + ")(" + b + ")))";
    };
    auto add = [&](const std::string &a, const std::string &b) {
      if (dt_is_float(n.dt)) return "(" + a + " + " + b + ")";
      std::string U = n.dt == DT::I64 ? "cc_u64" : "cc_u32";
      return "((" + T + ")((" + U + ")(" + a + ") + (" + U + ")(" + b + ")))";
    };
    int64_t nt = cdiv(K, 16);
    std::ostringstream k;
    k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "(" << params << ") {\n"
      << "  __shared__ " << T << " sa[16][17];\n"
      << "  __shared__ " << T << " sb[16][17];\n"
      << "  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;\n"
      << "  const int row = blockIdx.y * 16 + ty, col = blockIdx.x * 16 + tx;\n"
      << "  " << T << " acc = " << zero_of(n.dt) << ";\n"
      << "  for (int kt = 0; kt < " << nt << "; kt++) {\n"
      << "    const int ka = kt * 16 + tx, kb = kt * 16 + ty;\n"
      << "    sa[ty][tx] = (row < " << M << " && ka < " << K << ") ? " << fa.call_scalar("row * " + std::to_string(K) + " + ka")
      << " : " << zero_of(n.dt) << ";\n"
      << "    sb[ty][tx] = (kb < " << K << " && col < " << N << ") ? " << fb.call_scalar("kb * " + std::to_string(N) + " + col")
      << " : " << zero_of(n.dt) << ";\n"
      << "    __syncthreads();\n"
      << "#pragma unroll\n"
      << "    for (int q = 0; q < 16; q++) acc = " << add("acc", mul("sa[ty][q]", "sb[q][tx]")) << ";\n"
      << "    __syncthreads();\n"
      << "  }\n"
      << "  if (row < " << M << " && col < " << N << ") b" << out << "[row * " << N << " + col] = acc;\n"
      << "}\n";
    src << k.str();
    return {add_kernel(kname, args, (int)cdiv(N, 16), 256, "matmul_tiled", (int)cdiv(M, 16))};
  }

  // Uniform roots (broadcasts, and maps of them that do not use the
  // element index) whose buffer no other root's kernel reads (their
  // consumers compute the value instead; see Gen::elem) and that the graph
  // does not output: their kernels are dropped and their buffers never
  // allocated. The fusion plan itself is unchanged.
  void elide_unread_broadcasts(std::vector<std::vector<int>> &launches) {
    const bool remat = tune("remat_broadcast", 1) != 0;
    std::vector<char> dead_kernel(prog.kernels.size(), 0);
    bool any = false;
    for (size_t ri = 0; ri < plan.roots.size(); ri++) {
      const int r = plan.roots[ri];
      if (!(remat && gen.uniform(r)) && !gen.scatter_inline_.count(r)) continue;
      const int b = buf_of[r];
      bool needed = false;
      for (auto &o : g.outputs) needed |= o.second == r;
      for (size_t rj = 0; rj < launches.size() && !needed; rj++) {
        if (rj == ri) continue;
        for (int k : launches[rj])
          for (int a : prog.kernels[k].args) needed |= a == b;
      }
      if (needed) continue;
      prog.bufs[b].elided = true;
      for (int k : launches[ri]) dead_kernel[k] = 1;
      launches[ri].clear();
      any = true;
    }
    if (!any) return;
    std::vector<int> remap(prog.kernels.size(), -1);
    std::vector<KernelSpec> kept;
    for (size_t k = 0; k < prog.kernels.size(); k++)
      if (!dead_kernel[k]) {
        remap[k] = (int)kept.size();
        kept.push_back(prog.kernels[k]);
      }
    prog.kernels = kept;
    for (auto &l : launches)
      for (int &k : l) k = remap[k];
  }

  void run() {
    prog.name = g.name;
    buf_of.assign(g.ts.size(), -1);
    // Buffers: params first (in Graph.params order = topological order of
    // params), then the computed materialised nodes (lower.ml:977-990).
    for (size_t i = 0; i < g.ts.size(); i++)
      if (plan.materialized[i] && g.ts[i].kind == TK::Param)
        buf_of[i] = add_buf("p_" + g.ts[i].pname, g.ts[i].dt, g.ts[i].numel, BufRole::Param);
    for (size_t i = 0; i < g.ts.size(); i++)
      if (plan.materialized[i] && g.ts[i].kind != TK::Param)
        buf_of[i] = add_buf("t" + std::to_string(g.ts[i].id), g.ts[i].dt, g.ts[i].numel, BufRole::Computed);
    int ncomputed = (int)prog.bufs.size();
    src << kPrelude;
    // Roots gather(idx, h) over h = scatter_add(idx, ...) with the very same
    // index tensor read back through the scatter's partition
    // (scatter_gather_back=0 keeps them plain gathers).
    if (tune("scatter_gather_back", 1))
      for (int r : plan.roots) {
        const TNode &n = g.ts[r];
        if (n.kind != TK::Gather) continue;
        const int S = n.b;
        if (g.ts[S].kind == TK::Scatter && g.ts[S].a == n.a && !gbp_root_of.count(S)) gbp_root_of[S] = r;
      }
    // Scatters with an injective affine index in range are computed where
    // they are read (Gen::scatter_inline_; scatter_inline=0 reads their
    // buffers); their kernels and buffers go when nothing else reads them
    // (elide_unread_broadcasts). Config 5's gather adjoint, which puts each
    // path's adjoint at p * 64 + 63 of a 2^28-element tensor that one map
    // reads: 1 GiB written and read back.
    if (tune("scatter_inline", 1))
      for (int r : plan.roots) {
        const TNode &n = g.ts[r];
        if (n.kind != TK::Scatter || n.dt == DT::BOOL) continue;
        const int64_t M = n.numel, N = g.ts[n.a].numel;
        const Aff ia = aff_t(n.a);
        if (!ia.ok || ia.a == 0 || M <= 0 || N <= 0 || M > INT32_MAX - 4) continue;
        if (ia.a > INT32_MAX || ia.a < -INT32_MAX || ia.b > INT32_MAX || ia.b < -INT32_MAX) continue;
        const __int128 e0 = ia.b, e1 = (__int128)ia.a * (N - 1) + ia.b;
        if (std::min(e0, e1) < 0 || std::max(e0, e1) >= M) continue;
        gen.scatter_inline_[r] = {ia.a, ia.b};
      }
    // A reduction of a whole map output to one value, right after the map's
    // own root, is folded inside the map kernel when the map is light
    // (fuse_reduce=0: its own split reduction, reading the output back).
    // Measured step times, fused against not: saxpy 2^24 0.043 / 0.049 ms,
    // 2^28 0.52 / 0.67 ms; the degree-64 Horner map (VALU-bound, 48 lines or
    // more, as for map_unroll) 0.129 / 0.124 ms, since its waves then end
    // on the fold's dependent tail.
    //
    // The same when the reduction's input is an element-wise expression
    // (not materialised) of the map's output and of other tensors at the
    // same index (fuse_reduce_expr=0: its own split reduction): the map
    // kernel also loads those tensors, evaluates the expression on the
    // values it has just computed, and folds that. Its output is not read
    // back. The functions of both together stay under 48 lines. Config 5's
    // adjoint sums, sum(a * b) beside the map that makes a, are such.
    if (tune("fuse_reduce", 1)) {
      std::map<int, size_t> pos;
      for (size_t i = 0; i < plan.roots.size(); i++) pos[plan.roots[i]] = i;
      std::map<int, int> root_of_buf;
      for (int r : plan.roots) root_of_buf[buf_of[r]] = r;
      // m's kernel is the map template (a gather root takes it too, unless
      // it reads a scatter back through its partition)
      auto light = [&](int m, int64_t more, bool gathers) {
        const TNode &mn = g.ts[m];
        const bool gather = gathers && mn.kind == TK::Gather && !gbp_root_of.count(mn.b);
        if (mn.kind != TK::Map && mn.kind != TK::Map2 && !gather) return false;
        if (mn.numel < (1 << 16) || gen.uniform(m) || fused_red_of_map.count(m)) return false;
        const std::string code = gen.element_fn("fz_", m, true, true).code;
        return std::count(code.begin(), code.end(), '\n') + more < 48;
      };
      for (size_t ri = 0; ri < plan.roots.size(); ri++) {
        const int r = plan.roots[ri];
        const TNode &n = g.ts[r];
        if (n.kind != TK::Reduce || n.numel != 1 || n.dt == DT::BOOL) continue;
        if (plan.materialized[n.a]) {
          // the map's own output, the root just before
          const int m = n.a;
          if (ri == 0 || plan.roots[ri - 1] != m || g.ts[m].dt != n.dt || !light(m, 0, false)) continue;
          fused_red_of_map[m] = r;
          continue;
        }
        // An expression: folded in the kernel of the last root among the
        // tensors it reads (every other one is ready by then), when that
        // root is a map whose output it reads at its own index.
        if (!tune("fuse_reduce_expr", 1)) continue;
        const ElemFn fe = gen.element_fn("fz_", n.a, false, true);
        int m = -1;
        bool known = true;
        for (const auto *v : {&fe.ident, &fe.ptrs})
          for (int b : *v) {
            const auto ro = root_of_buf.find(b);
            if (ro == root_of_buf.end()) {
              known = known && prog.bufs[b].role == BufRole::Param;
              continue;
            }
            if (m < 0 || pos[ro->second] > pos[m]) m = ro->second;
          }
        if (!known || m < 0 || pos[m] > ri || g.ts[m].numel != g.ts[n.a].numel) continue;
        const int mb = buf_of[m];
        if (std::find(fe.ident.begin(), fe.ident.end(), mb) == fe.ident.end() ||
            std::find(fe.ptrs.begin(), fe.ptrs.end(), mb) != fe.ptrs.end())
          continue;
        if (!light(m, std::count(fe.code.begin(), fe.code.end(), '\n'), true)) continue;
        fused_red_of_map[m] = r;
      }
    }
    find_sibling_groups();
    find_rowlast_gathers();
    // the side buffers are computed buffers too: allocated with the others
    // for the program's lifetime
    for (size_t b = ncomputed; b < prog.bufs.size(); b++)
      if (prog.bufs[b].role != BufRole::Computed) throw Failure("Lower: a scratch buffer before the roots");
    ncomputed = (int)prog.bufs.size();
    std::vector<std::vector<int>> launches;
    std::vector<std::vector<int>> scratch_of;
    for (int r : plan.roots) {
      size_t before = prog.bufs.size();
      std::vector<int> ks;
      if (sib_member.count(r)) {
        // lowered with its group's lead
      } else if (sib_lead.count(r)) {
        const int sc = sib_lead[r];
        ks = lower_scan(sc, sib_reds[sc]);
        attribute_group_bytes(sc, sib_reds[sc], ks);
      } else switch (g.ts[r].kind) {
        case TK::Gather: {
          auto it = gather_back.find(g.ts[r].b);
          auto ro = gbp_root_of.find(g.ts[r].b);
          ks = it != gather_back.end() && ro != gbp_root_of.end() && ro->second == r ? lower_gather_back(r, it->second)
                                                                                    : lower_map(r);
          break;
        }
        case TK::Map:
        case TK::Map2:
        case TK::Iota:
        case TK::Reshape:
        case TK::Broadcast: ks = lower_map(r); break;
        case TK::Reduce: ks = lower_reduce(r); break;
        case TK::Scan: ks = lower_scan(r); break;
        case TK::Scatter: ks = lower_scatter(r); break;
        case TK::Matmul: ks = lower_matmul(r); break;
        default: throw Failure("Lower: a Param never gets a kernel");
      }
      if (!sib_member.count(r) && !sib_lead.count(r)) attribute_bytes(r, ks);
      std::vector<int> sc;
      for (size_t b = before; b < prog.bufs.size(); b++)
        if (prog.bufs[b].role == BufRole::Scratch) sc.push_back((int)b);
      launches.push_back(ks);
      scratch_of.push_back(sc);
    }
    prog.source = src.str();
    elide_unread_broadcasts(launches);
    for (size_t i = 0; i < g.ts.size(); i++)
      if (g.ts[i].kind == TK::Param) prog.params.push_back({g.ts[i].pname, g.ts[i].dt, g.ts[i].shape, buf_of[i]});
    for (auto &o : g.outputs) prog.outputs.push_back({o.first, g.ts[o.second].dt, g.ts[o.second].shape, buf_of[o.second]});
    // Host plan.
    for (int b = 0; b < ncomputed; b++)
      if (!prog.bufs[b].elided) prog.plan.push_back({OpK::Alloc, b, -1, ""});
    if (prog.err_buf >= 0) prog.plan.push_back({OpK::Alloc, prog.err_buf, -1, ""});
    for (auto &p : prog.params) prog.plan.push_back({OpK::Upload, p.buf, -1, p.name});
    for (size_t r = 0; r < launches.size(); r++) {
      for (int b : scratch_of[r]) prog.plan.push_back({OpK::Alloc, b, -1, ""});
      for (int k : launches[r]) prog.plan.push_back({OpK::Launch, -1, k, ""});
      for (int b : scratch_of[r])
        if (!free_after.count(b)) prog.plan.push_back({OpK::Free, b, -1, ""});
      for (auto &fa : free_after)
        if (fa.second == plan.roots[r]) prog.plan.push_back({OpK::Free, fa.first, -1, ""});
    }
    for (auto &o : prog.outputs) prog.plan.push_back({OpK::Download, o.buf, -1, o.name});
    for (int b = 0; b < ncomputed; b++)
      if (!prog.bufs[b].elided) prog.plan.push_back({OpK::Free, b, -1, ""});
    if (prog.err_buf >= 0) prog.plan.push_back({OpK::Free, prog.err_buf, -1, ""});
  }
};

}  // namespace

int64_t tune_knob(const char *key, int64_t dflt) { return tune(key, dflt); }

ProgramIR lower_program(const Graph &g) {
  Lowering l(g);
  l.run();
  // A map root whose reduction folds in its kernel may have no reader
  // left: a tensor materialised because the reduction's expression uses it
  // twice (config 5's last adjoint map, 1 GiB). Lowered again, its kernel
  // stores only the partials (skip_unread_stores=0 keeps the store).
  if (tune("skip_unread_stores", 1)) {
    std::set<int> unread;
    for (auto &fr : l.fused_red_of_map) {
      const int m = fr.first, b = l.buf_of[m];
      const std::string own = "k_" + std::to_string(g.ts[m].id);
      bool read = l.gen.rowlast_.count(m) > 0;
      for (auto &o : g.outputs) read |= o.second == m;
      for (const KernelSpec &k : l.prog.kernels) {
        if (read) break;
        if (k.name == own) continue;
        for (int a : k.args) read |= a == b;
      }
      if (!read) unread.insert(m);
    }
    if (!unread.empty()) {
      Lowering l2(g);
      l2.no_store = unread;
      l2.run();
      return l2.prog;
    }
  }
  return l.prog;
}

std::string plan_to_string(const ProgramIR &p) {
  std::ostringstream os;
  os << "program " << p.name << "\n";
  for (size_t i = 0; i < p.bufs.size(); i++) {
    const BufSpec &b = p.bufs[i];
    static const char *roles[] = {"param", "computed", "scratch", "err"};
    os << "buffer " << i << " " << b.name << " " << dt_name(b.dt) << " " << b.numel << " "
       << (b.elided ? "elided" : roles[(int)b.role]) << "\n";
  }
  for (auto &k : p.kernels) {
    os << "kernel " << k.name << " " << k.role << " grid " << k.grid << " " << k.grid_y << " block " << k.block
       << " bytes " << k.algo_bytes << " moved " << k.moved_bytes << " args";
    for (int a : k.args) os << " " << a;
    os << "\n";
  }
  for (auto &o : p.plan) {
    switch (o.kind) {
      case OpK::Alloc: os << "alloc " << p.bufs[o.buf].name << "\n"; break;
      case OpK::Upload: os << "upload " << o.name << " " << p.bufs[o.buf].name << "\n"; break;
      case OpK::Launch: os << "launch " << p.kernels[o.kernel].name << "\n"; break;
      case OpK::Download: os << "download " << o.name << " " << p.bufs[o.buf].name << "\n"; break;
      case OpK::Free: os << "free " << p.bufs[o.buf].name << "\n"; break;
    }
  }
  return os.str();
}

}  // namespace cchip
