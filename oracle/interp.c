/*
 * CPU oracle: a single-threaded C restatement of the reference interpreter,
 * lib/backend_interp/cudacaml_backend_interp.ml (Backend_interp).
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (cudacaml_amd/) may
 * import, link or run this file or the library built from it; only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and only
 * as the checker.
 *
 * It reads the text wire format that cudacaml_amd/ir.py writes (one graph;
 * expression DAG, tensor nodes in topological order, outputs) and follows
 * the interpreter rule for rule:
 *
 *   R1  every F32 binop/unop is computed in double and rounded once
 *       (round_f32, cudacaml_backend_interp.ml:34-36,61,160)
 *   R2  Reduce is a strictly sequential left fold per row from init, an
 *       empty row yields init; Scan is inclusive and restarts per row
 *       (:335-370)
 *   R3  an F32 Const is the double itself, never rounded (:246)
 *   R4  integers wrap; division truncates toward zero and raises on zero;
 *       shift counts are masked and Shr is logical (:56-91)
 *   R5  Min/Max follow OCaml's Float.min/Float.max: NaN if either operand
 *       is NaN, and min(-0,+0) = -0, max(-0,+0) = +0 (:48-49)
 *   R6  float->int casts truncate through int64 then wrap to int32;
 *       int->f32 goes int -> double -> f32 (:198-237)
 *   R7  erfinv: Giles' single-precision polynomial as the starting point,
 *       then two Newton steps on erf (:94-143). The method and its
 *       coefficients are published: M. Giles, "Approximating the erfinv
 *       function", GPU Computing Gems Jade Edition, 2011.
 *   R8  Scatter_add is a sequential left fold in source order; Gather and
 *       Scatter_add raise on an index out of range (:371-406)
 *   R9  Matmul: acc = round(acc + round(a*b)), p ascending, no FMA (:407-433)
 *   R10 Index is the flat element index; inside a Reduce/Scan combine it
 *       is the flat source index (:243-257, :345-349)
 *
 * Evaluation order differs in one harmless way: tensor nodes are computed
 * in topological order rather than by memoised recursion from the outputs
 * (every node in the order is reachable from an output, so the same nodes
 * are computed), and a shared sub-expression is evaluated once per element
 * rather than once per use (expressions are pure). Intermediate tensors are
 * freed after their last use.
 */
#define _GNU_SOURCE
#include <math.h>
#include <setjmp.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

enum { DT_F32 = 0, DT_F64 = 1, DT_I32 = 2, DT_I64 = 3, DT_BOOL = 4 };

enum {
  X_CONST, X_ARG, X_INDEX, X_BIN, X_UN, X_CMP, X_LOGIC, X_NOT, X_SELECT, X_CAST
};
enum { B_ADD, B_SUB, B_MUL, B_DIV, B_MIN, B_MAX, B_AND, B_OR, B_XOR, B_SHL, B_SHR };
enum { U_NEG, U_SQRT, U_EXP, U_LOG, U_ABS, U_SIN, U_COS, U_ERF, U_ERFINV };
enum { C_EQ, C_NE, C_LT, C_LE, C_GT, C_GE };
enum { L_AND, L_OR };
enum {
  T_PARAM, T_IOTA, T_MAP, T_MAP2, T_REDUCE, T_SCAN, T_GATHER, T_SCATTER,
  T_MATMUL, T_RESHAPE, T_BROADCAST
};

#define MAX_RANK 8

typedef struct {
  int kind, dt, op;
  int a, b, c; /* positions of operands */
  double f;
  int64_t i;
  int arg;
} xnode;

typedef struct {
  int kind, dt, rank;
  int64_t dims[MAX_RANK];
  int64_t numel;
  int a, b;       /* positions of operand tensors */
  int init, body; /* positions of expressions */
  char *pname;
} tnode;

typedef struct {
  int64_t *keys;
  int *vals;
  int64_t cap, count;
} idmap;

typedef struct orc_graph {
  char *name;
  int nx, capx;
  xnode *xs;
  int nt, capt;
  tnode *ts;
  int no;
  char **onames;
  int *otid;
  idmap xmap, tmap;
} orc_graph;

typedef union {
  double f;
  int64_t i;
} val;

typedef struct {
  int dt, rank;
  int64_t dims[MAX_RANK];
  int64_t n;
  void *data;
  int owned;
} tval;

typedef struct orc_result {
  int count;
  char **names;
  tval *vals;
} orc_result;

/* ------------------------------------------------------------------ */
/* errors                                                              */
/* ------------------------------------------------------------------ */

static __thread jmp_buf *err_jmp;
static __thread char err_msg[1024];

static __attribute__((noreturn, format(printf, 1, 2))) void fail(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(err_msg, sizeof err_msg, fmt, ap);
  va_end(ap);
  longjmp(*err_jmp, 1);
}

static void *xmalloc(size_t n) {
  void *p = malloc(n ? n : 1);
  if (!p) fail("oracle: out of host memory (%zu bytes)", n);
  return p;
}

static void *xcalloc(size_t n, size_t sz) {
  void *p = calloc(n ? n : 1, sz ? sz : 1);
  if (!p) fail("oracle: out of host memory (%zu bytes)", n * sz);
  return p;
}

/* ------------------------------------------------------------------ */
/* id map                                                              */
/* ------------------------------------------------------------------ */

static void idmap_grow(idmap *m);

static int64_t idmap_slot(const idmap *m, int64_t k) {
  return (int64_t)(((uint64_t)k * 0x9E3779B97F4A7C15ull) >> 11) % m->cap;
}

static void idmap_put(idmap *m, int64_t k, int v) {
  if (k <= 0) fail("oracle: node ids must be positive, got %lld", (long long)k);
  if ((m->count + 1) * 2 > m->cap) idmap_grow(m);
  for (int64_t s = idmap_slot(m, k);; s = (s + 1) % m->cap) {
    if (m->keys[s] == 0) {
      m->keys[s] = k;
      m->vals[s] = v;
      m->count++;
      return;
    }
    if (m->keys[s] == k) fail("oracle: duplicate node id %lld", (long long)k);
  }
}

static int idmap_get(const idmap *m, int64_t k) {
  if (m->cap == 0) return -1;
  for (int64_t s = idmap_slot(m, k);; s = (s + 1) % m->cap) {
    if (m->keys[s] == 0) return -1;
    if (m->keys[s] == k) return m->vals[s];
  }
}

static void idmap_grow(idmap *m) {
  int64_t oc = m->cap;
  int64_t *ok = m->keys;
  int *ov = m->vals;
  m->cap = oc ? oc * 2 : 1024;
  m->count = 0;
  m->keys = (int64_t *)xcalloc((size_t)m->cap, sizeof(int64_t));
  m->vals = (int *)xcalloc((size_t)m->cap, sizeof(int));
  for (int64_t i = 0; i < oc; i++)
    if (ok[i]) idmap_put(m, ok[i], ov[i]);
  free(ok);
  free(ov);
}

/* ------------------------------------------------------------------ */
/* wire parser                                                         */
/* ------------------------------------------------------------------ */

typedef struct {
  const char *p;
  int line;
} lexer;

static int at_eol(lexer *lx) {
  while (*lx->p == ' ' || *lx->p == '\t' || *lx->p == '\r') lx->p++;
  return *lx->p == '\n' || *lx->p == 0;
}

static void next_line(lexer *lx) {
  while (*lx->p && *lx->p != '\n') lx->p++;
  if (*lx->p == '\n') {
    lx->p++;
    lx->line++;
  }
}

static char *token(lexer *lx) {
  if (at_eol(lx)) fail("oracle: wire line %d: missing field", lx->line);
  const char *s = lx->p;
  while (*lx->p && *lx->p != ' ' && *lx->p != '\t' && *lx->p != '\n' && *lx->p != '\r') lx->p++;
  size_t n = (size_t)(lx->p - s);
  char *t = (char *)xmalloc(n + 1);
  memcpy(t, s, n);
  t[n] = 0;
  return t;
}

static int64_t tok_int(lexer *lx) {
  char *t = token(lx);
  char *end;
  long long v = strtoll(t, &end, 10);
  if (*end) fail("oracle: wire line %d: bad integer '%s'", lx->line, t);
  free(t);
  return (int64_t)v;
}

static int tok_is(const char *t, const char *w) { return strcmp(t, w) == 0; }

static int parse_dtype(lexer *lx) {
  char *t = token(lx);
  int d = -1;
  if (tok_is(t, "f32")) d = DT_F32;
  else if (tok_is(t, "f64")) d = DT_F64;
  else if (tok_is(t, "i32")) d = DT_I32;
  else if (tok_is(t, "i64")) d = DT_I64;
  else if (tok_is(t, "bool")) d = DT_BOOL;
  if (d < 0) fail("oracle: wire line %d: bad dtype '%s'", lx->line, t);
  free(t);
  return d;
}

static char *unescape(const char *t) {
  size_t n = strlen(t);
  char *o = (char *)xmalloc(n + 1);
  size_t j = 0;
  if (strcmp(t, "%") == 0) {
    o[0] = 0;
    return o;
  }
  for (size_t i = 0; i < n; i++) {
    if (t[i] == '%' && i + 2 < n + 1 && t[i + 1] && t[i + 2]) {
      char hx[3] = {t[i + 1], t[i + 2], 0};
      o[j++] = (char)strtol(hx, NULL, 16);
      i += 2;
    } else {
      o[j++] = t[i];
    }
  }
  o[j] = 0;
  return o;
}

static int lookup_x(orc_graph *g, lexer *lx) {
  int64_t id = tok_int(lx);
  int p = idmap_get(&g->xmap, id);
  if (p < 0) fail("oracle: wire line %d: unknown expression %lld", lx->line, (long long)id);
  return p;
}

static int lookup_t(orc_graph *g, lexer *lx) {
  int64_t id = tok_int(lx);
  int p = idmap_get(&g->tmap, id);
  if (p < 0) fail("oracle: wire line %d: unknown tensor %lld", lx->line, (long long)id);
  return p;
}

static int op_index(const char *t, const char *const *names, int n, lexer *lx) {
  for (int i = 0; i < n; i++)
    if (tok_is(t, names[i])) return i;
  fail("oracle: wire line %d: bad operator '%s'", lx->line, t);
  return -1;
}

static const char *const BIN_NAMES[] = {"add", "sub", "mul", "div", "min", "max",
                                        "and", "or",  "xor", "shl", "shr"};
static const char *const UN_NAMES[] = {"neg", "sqrt", "exp", "log", "abs",
                                       "sin", "cos",  "erf", "erfinv"};
static const char *const CMP_NAMES[] = {"eq", "ne", "lt", "le", "gt", "ge"};
static const char *const LOGIC_NAMES[] = {"and", "or"};

static void parse_expr(orc_graph *g, lexer *lx) {
  int64_t id = tok_int(lx);
  char *kind = token(lx);
  xnode x;
  memset(&x, 0, sizeof x);
  x.dt = parse_dtype(lx);
  x.a = x.b = x.c = -1;
  if (tok_is(kind, "const")) {
    x.kind = X_CONST;
    char *t = token(lx);
    if (x.dt == DT_F32 || x.dt == DT_F64) {
      uint64_t bits = strtoull(t, NULL, 16);
      memcpy(&x.f, &bits, 8);
    } else {
      x.i = strtoll(t, NULL, 10);
    }
    free(t);
  } else if (tok_is(kind, "arg")) {
    x.kind = X_ARG;
    x.arg = (int)tok_int(lx);
  } else if (tok_is(kind, "index")) {
    x.kind = X_INDEX;
  } else if (tok_is(kind, "bin") || tok_is(kind, "cmp") || tok_is(kind, "logic")) {
    char *op = token(lx);
    if (tok_is(kind, "bin")) {
      x.kind = X_BIN;
      x.op = op_index(op, BIN_NAMES, 11, lx);
    } else if (tok_is(kind, "cmp")) {
      x.kind = X_CMP;
      x.op = op_index(op, CMP_NAMES, 6, lx);
    } else {
      x.kind = X_LOGIC;
      x.op = op_index(op, LOGIC_NAMES, 2, lx);
    }
    free(op);
    x.a = lookup_x(g, lx);
    x.b = lookup_x(g, lx);
  } else if (tok_is(kind, "un")) {
    char *op = token(lx);
    x.kind = X_UN;
    x.op = op_index(op, UN_NAMES, 9, lx);
    free(op);
    x.a = lookup_x(g, lx);
  } else if (tok_is(kind, "not")) {
    x.kind = X_NOT;
    x.a = lookup_x(g, lx);
  } else if (tok_is(kind, "cast")) {
    x.kind = X_CAST;
    x.a = lookup_x(g, lx);
  } else if (tok_is(kind, "select")) {
    x.kind = X_SELECT;
    x.a = lookup_x(g, lx);
    x.b = lookup_x(g, lx);
    x.c = lookup_x(g, lx);
  } else {
    fail("oracle: wire line %d: bad expression kind '%s'", lx->line, kind);
  }
  free(kind);
  if (g->nx == g->capx) {
    g->capx = g->capx ? g->capx * 2 : 256;
    xnode *nx = (xnode *)realloc(g->xs, (size_t)g->capx * sizeof(xnode));
    if (!nx) fail("oracle: out of host memory");
    g->xs = nx;
  }
  g->xs[g->nx] = x;
  idmap_put(&g->xmap, id, g->nx);
  g->nx++;
}

static void parse_tensor(orc_graph *g, lexer *lx) {
  int64_t id = tok_int(lx);
  char *kind = token(lx);
  tnode t;
  memset(&t, 0, sizeof t);
  t.dt = parse_dtype(lx);
  t.rank = (int)tok_int(lx);
  if (t.rank < 0 || t.rank > MAX_RANK) fail("oracle: wire line %d: rank %d unsupported", lx->line, t.rank);
  t.numel = 1;
  for (int i = 0; i < t.rank; i++) {
    t.dims[i] = tok_int(lx);
    if (t.dims[i] < 0) fail("oracle: wire line %d: negative extent", lx->line);
    /* checked before multiplying: no extent list can wrap the count */
    if (t.dims[i] > ((int64_t)1 << 62) || (t.dims[i] && t.numel > ((int64_t)1 << 62) / t.dims[i]))
      fail("oracle: wire line %d: too many elements", lx->line);
    t.numel *= t.dims[i];
  }
  t.a = t.b = t.init = t.body = -1;
  if (tok_is(kind, "param")) {
    t.kind = T_PARAM;
    char *n = token(lx);
    t.pname = unescape(n);
    free(n);
  } else if (tok_is(kind, "iota")) {
    t.kind = T_IOTA;
  } else if (tok_is(kind, "map")) {
    t.kind = T_MAP;
    t.a = lookup_t(g, lx);
    t.body = lookup_x(g, lx);
  } else if (tok_is(kind, "map2")) {
    t.kind = T_MAP2;
    t.a = lookup_t(g, lx);
    t.b = lookup_t(g, lx);
    t.body = lookup_x(g, lx);
  } else if (tok_is(kind, "reduce") || tok_is(kind, "scan")) {
    t.kind = tok_is(kind, "reduce") ? T_REDUCE : T_SCAN;
    t.a = lookup_t(g, lx);
    t.init = lookup_x(g, lx);
    t.body = lookup_x(g, lx);
  } else if (tok_is(kind, "gather") || tok_is(kind, "scatter_add") || tok_is(kind, "matmul")) {
    t.kind = tok_is(kind, "gather") ? T_GATHER : tok_is(kind, "matmul") ? T_MATMUL : T_SCATTER;
    t.a = lookup_t(g, lx);
    t.b = lookup_t(g, lx);
  } else if (tok_is(kind, "reshape") || tok_is(kind, "broadcast")) {
    t.kind = tok_is(kind, "reshape") ? T_RESHAPE : T_BROADCAST;
    t.a = lookup_t(g, lx);
  } else {
    fail("oracle: wire line %d: bad tensor kind '%s'", lx->line, kind);
  }
  free(kind);
  if (g->nt == g->capt) {
    g->capt = g->capt ? g->capt * 2 : 64;
    tnode *nt = (tnode *)realloc(g->ts, (size_t)g->capt * sizeof(tnode));
    if (!nt) fail("oracle: out of host memory");
    g->ts = nt;
  }
  g->ts[g->nt] = t;
  idmap_put(&g->tmap, id, g->nt);
  g->nt++;
}

void orc_free(orc_graph *g) {
  if (!g) return;
  free(g->name);
  free(g->xs);
  for (int i = 0; i < g->nt; i++) free(g->ts[i].pname);
  free(g->ts);
  for (int i = 0; i < g->no; i++) free(g->onames[i]);
  free(g->onames);
  free(g->otid);
  free(g->xmap.keys);
  free(g->xmap.vals);
  free(g->tmap.keys);
  free(g->tmap.vals);
  free(g);
}

orc_graph *orc_parse(const char *text, char *err, int errlen) {
  jmp_buf jb;
  jmp_buf *saved = err_jmp;
  orc_graph *volatile g = (orc_graph *)calloc(1, sizeof(orc_graph));
  if (!g) {
    snprintf(err, (size_t)errlen, "oracle: out of host memory");
    return NULL;
  }
  err_jmp = &jb;
  if (setjmp(jb)) {
    err_jmp = saved;
    snprintf(err, (size_t)errlen, "%s", err_msg);
    orc_free(g);
    return NULL;
  }
  lexer lx = {text, 1};
  char *h = token(&lx);
  if (!tok_is(h, "cchip-graph")) fail("oracle: not a cchip-graph text");
  free(h);
  if (tok_int(&lx) != 1) fail("oracle: unsupported wire version");
  char *nm = token(&lx);
  g->name = unescape(nm);
  free(nm);
  next_line(&lx);
  int ended = 0;
  while (*lx.p) {
    if (at_eol(&lx)) {
      next_line(&lx);
      continue;
    }
    char *tag = token(&lx);
    if (tok_is(tag, "x")) parse_expr(g, &lx);
    else if (tok_is(tag, "t")) parse_tensor(g, &lx);
    else if (tok_is(tag, "o")) {
      char *n = token(&lx);
      g->onames = (char **)realloc(g->onames, (size_t)(g->no + 1) * sizeof(char *));
      g->otid = (int *)realloc(g->otid, (size_t)(g->no + 1) * sizeof(int));
      g->onames[g->no] = unescape(n);
      free(n);
      g->otid[g->no] = lookup_t(g, &lx);
      g->no++;
    } else if (tok_is(tag, "end")) {
      ended = 1;
      free(tag);
      break;
    } else {
      fail("oracle: wire line %d: bad tag '%s'", lx.line, tag);
    }
    free(tag);
    if (!at_eol(&lx)) fail("oracle: wire line %d: trailing fields", lx.line);
    next_line(&lx);
  }
  if (!ended) fail("oracle: wire text has no 'end'");
  if (g->no == 0) fail("oracle: graph has no output");
  err_jmp = saved;
  return g;
}

int orc_num_params(const orc_graph *g) {
  int n = 0;
  for (int i = 0; i < g->nt; i++) n += g->ts[i].kind == T_PARAM;
  return n;
}

/* ------------------------------------------------------------------ */
/* scalar semantics                                                    */
/* ------------------------------------------------------------------ */

static double round_f32(double x) { return (double)(float)x; }

/* OCaml's Float.min / Float.max: NaN wins, and -0 orders below +0. */
static double ocaml_min(double x, double y) {
  if (isnan(x) || isnan(y)) return NAN;
  if (x < y) return x;
  if (y < x) return y;
  return signbit(x) ? x : y;
}

static double ocaml_max(double x, double y) {
  if (isnan(x) || isnan(y)) return NAN;
  if (x > y) return x;
  if (y > x) return y;
  return signbit(x) ? y : x;
}

static double float_binop(int op, double x, double y) {
  switch (op) {
    case B_ADD: return x + y;
    case B_SUB: return x - y;
    case B_MUL: return x * y;
    case B_DIV: return x / y;
    case B_MIN: return ocaml_min(x, y);
    case B_MAX: return ocaml_max(x, y);
    case B_AND: fail("Backend_interp: bit_and on a float dtype");
    case B_OR: fail("Backend_interp: bit_or on a float dtype");
    case B_XOR: fail("Backend_interp: bit_xor on a float dtype");
    case B_SHL: fail("Backend_interp: shl on a float dtype");
    default: fail("Backend_interp: shr on a float dtype");
  }
  return 0;
}

static int32_t i32_binop(int op, int32_t x, int32_t y) {
  uint32_t ux = (uint32_t)x, uy = (uint32_t)y;
  switch (op) {
    case B_ADD: return (int32_t)(ux + uy);
    case B_SUB: return (int32_t)(ux - uy);
    case B_MUL: return (int32_t)(ux * uy);
    case B_DIV:
      if (y == 0) fail("Division_by_zero");
      if (y == -1) return (int32_t)(0u - ux);
      return x / y;
    case B_MIN: return x < y ? x : y;
    case B_MAX: return x > y ? x : y;
    case B_AND: return (int32_t)(ux & uy);
    case B_OR: return (int32_t)(ux | uy);
    case B_XOR: return (int32_t)(ux ^ uy);
    case B_SHL: return (int32_t)(ux << (uy & 31u));
    default: return (int32_t)(ux >> (uy & 31u));
  }
}

static int64_t i64_binop(int op, int64_t x, int64_t y) {
  uint64_t ux = (uint64_t)x, uy = (uint64_t)y;
  switch (op) {
    case B_ADD: return (int64_t)(ux + uy);
    case B_SUB: return (int64_t)(ux - uy);
    case B_MUL: return (int64_t)(ux * uy);
    case B_DIV:
      if (y == 0) fail("Division_by_zero");
      if (y == -1) return (int64_t)(0ull - ux);
      return x / y;
    case B_MIN: return x < y ? x : y;
    case B_MAX: return x > y ? x : y;
    case B_AND: return (int64_t)(ux & uy);
    case B_OR: return (int64_t)(ux | uy);
    case B_XOR: return (int64_t)(ux ^ uy);
    case B_SHL: return (int64_t)(ux << (uy & 63u));
    default: return (int64_t)(ux >> (uy & 63u));
  }
}

/* Giles (2011), single-precision branch coefficients, as a starting point
   for two Newton steps in double. */
static double erfinv_guess(double x) {
  double w = -log((1.0 - x) * (1.0 + x));
  double p;
  if (w < 5.0) {
    w = w - 2.5;
    p = 2.81022636e-08;
    p = 3.43273939e-07 + p * w;
    p = -3.5233877e-06 + p * w;
    p = -4.39150654e-06 + p * w;
    p = 0.00021858087 + p * w;
    p = -0.00125372503 + p * w;
    p = -0.00417768164 + p * w;
    p = 0.246640727 + p * w;
    p = 1.50140941 + p * w;
  } else {
    w = sqrt(w) - 3.0;
    p = -0.000200214257;
    p = 0.000100950558 + p * w;
    p = 0.00134934322 + p * w;
    p = -0.00367342844 + p * w;
    p = 0.00573950773 + p * w;
    p = -0.0076224613 + p * w;
    p = 0.00943887047 + p * w;
    p = 1.00167406 + p * w;
    p = 2.83297682 + p * w;
  }
  return p * x;
}

double orc_erfinv(double x) {
  if (isnan(x)) return x;
  if (x == 1.0) return INFINITY;
  if (x == -1.0) return -INFINITY;
  if (fabs(x) > 1.0) return NAN;
  if (x == 0.0) return x;
  const double two_over_sqrt_pi = 2.0 / sqrt(M_PI);
  double y = erfinv_guess(x);
  for (int k = 0; k < 2; k++) {
    double d = two_over_sqrt_pi * exp(-(y * y));
    if (d != 0.0) y = y - (erf(y) - x) / d;
  }
  return y;
}

static double float_unop(int op, double x) {
  switch (op) {
    case U_NEG: return -x;
    case U_SQRT: return sqrt(x);
    case U_EXP: return exp(x);
    case U_LOG: return log(x);
    case U_ABS: return fabs(x);
    case U_SIN: return sin(x);
    case U_COS: return cos(x);
    case U_ERF: return erf(x);
    default: return orc_erfinv(x);
  }
}

static const char *const UN_LABEL[] = {"neg", "sqrt", "exp", "log", "abs", "sin", "cos", "erf", "erfinv"};

/* Int64.of_float: truncation toward zero; out-of-range and NaN give
   0x8000000000000000 as the x86-64 conversion does. */
static int64_t int64_of_float(double x) {
  if (isnan(x) || x >= 9223372036854775808.0 || x < -9223372036854775808.0)
    return INT64_MIN;
  return (int64_t)x;
}

static val cast_val(int from, int to, val v) {
  val r;
  r.i = 0;
  if (from == to) return v;
  switch (from) {
    case DT_F32:
    case DT_F64:
      switch (to) {
        case DT_F32: r.f = round_f32(v.f); break;
        case DT_F64: r.f = v.f; break;
        case DT_I32: r.i = (int32_t)(uint32_t)(uint64_t)int64_of_float(v.f); break;
        case DT_I64: r.i = int64_of_float(v.f); break;
        default: r.i = v.f != 0.0; break;
      }
      break;
    case DT_I32:
    case DT_I64:
      switch (to) {
        case DT_F32: r.f = round_f32((double)v.i); break;
        case DT_F64: r.f = (double)v.i; break;
        case DT_I32: r.i = (int32_t)(uint32_t)(uint64_t)v.i; break;
        case DT_I64: r.i = v.i; break;
        default: r.i = v.i != 0; break;
      }
      break;
    default: /* bool */
      switch (to) {
        case DT_F32:
        case DT_F64: r.f = v.i ? 1.0 : 0.0; break;
        default: r.i = v.i ? 1 : 0; break;
      }
  }
  return r;
}

static int is_floatdt(int d) { return d == DT_F32 || d == DT_F64; }

/* ------------------------------------------------------------------ */
/* expression evaluation: lazy, memoised per element                   */
/* ------------------------------------------------------------------ */

typedef struct {
  const orc_graph *g;
  val *memo;
  uint64_t *stamp;
  uint64_t cur;
  val env[2];
  int envdt[2];
  int nenv;
  int64_t index;
} evalctx;

static val eval(evalctx *c, int p);

static val eval_raw(evalctx *c, int p) {
  const xnode *x = &c->g->xs[p];
  val r;
  r.i = 0;
  switch (x->kind) {
    case X_CONST:
      if (is_floatdt(x->dt)) r.f = x->f;
      else r.i = x->i;
      return r;
    case X_ARG:
      if (x->arg < 0 || x->arg >= c->nenv) fail("Backend_interp: Arg %d is unbound", x->arg);
      if (c->envdt[x->arg] != x->dt) fail("Backend_interp: Arg %d has the wrong dtype", x->arg);
      return c->env[x->arg];
    case X_INDEX:
      r.i = (int32_t)c->index;
      return r;
    case X_BIN: {
      val a = eval(c, x->a), b = eval(c, x->b);
      switch (x->dt) {
        case DT_F32: r.f = round_f32(float_binop(x->op, a.f, b.f)); break;
        case DT_F64: r.f = float_binop(x->op, a.f, b.f); break;
        case DT_I32: r.i = i32_binop(x->op, (int32_t)a.i, (int32_t)b.i); break;
        case DT_I64: r.i = i64_binop(x->op, a.i, b.i); break;
        default: fail("Backend_interp: binop on bool");
      }
      return r;
    }
    case X_UN: {
      val a = eval(c, x->a);
      switch (x->dt) {
        case DT_F32: r.f = round_f32(float_unop(x->op, a.f)); break;
        case DT_F64: r.f = float_unop(x->op, a.f); break;
        case DT_I32:
          if (x->op == U_NEG) r.i = (int32_t)(0u - (uint32_t)a.i);
          else if (x->op == U_ABS) r.i = a.i < 0 ? (int32_t)(0u - (uint32_t)a.i) : a.i;
          else fail("Backend_interp: %s on i32", UN_LABEL[x->op]);
          break;
        case DT_I64:
          if (x->op == U_NEG) r.i = (int64_t)(0ull - (uint64_t)a.i);
          else if (x->op == U_ABS) r.i = a.i < 0 ? (int64_t)(0ull - (uint64_t)a.i) : a.i;
          else fail("Backend_interp: %s on i64", UN_LABEL[x->op]);
          break;
        default: fail("Backend_interp: unop on bool");
      }
      return r;
    }
    case X_CMP: {
      int od = c->g->xs[x->a].dt;
      val a = eval(c, x->a), b = eval(c, x->b);
      int res;
      if (is_floatdt(od)) {
        double u = a.f, v = b.f;
        switch (x->op) {
          case C_EQ: res = u == v; break;
          case C_NE: res = u != v; break;
          case C_LT: res = u < v; break;
          case C_LE: res = u <= v; break;
          case C_GT: res = u > v; break;
          default: res = u >= v; break;
        }
      } else {
        int64_t u = a.i, v = b.i;
        switch (x->op) {
          case C_EQ: res = u == v; break;
          case C_NE: res = u != v; break;
          case C_LT: res = u < v; break;
          case C_LE: res = u <= v; break;
          case C_GT: res = u > v; break;
          default: res = u >= v; break;
        }
      }
      r.i = res;
      return r;
    }
    case X_LOGIC: {
      val a = eval(c, x->a);
      if (x->op == L_AND) r.i = a.i ? (eval(c, x->b).i != 0) : 0;
      else r.i = a.i ? 1 : (eval(c, x->b).i != 0);
      return r;
    }
    case X_NOT:
      r.i = !eval(c, x->a).i;
      return r;
    case X_SELECT:
      return eval(c, x->a).i ? eval(c, x->b) : eval(c, x->c);
    default: /* X_CAST */
      return cast_val(c->g->xs[x->a].dt, x->dt, eval(c, x->a));
  }
}

static val eval(evalctx *c, int p) {
  if (c->stamp[p] == c->cur) return c->memo[p];
  val v = eval_raw(c, p);
  c->memo[p] = v;
  c->stamp[p] = c->cur;
  return v;
}

static val eval_at(evalctx *c, int p, int64_t index) {
  c->cur++;
  c->index = index;
  return eval(c, p);
}

/* ------------------------------------------------------------------ */
/* tensor values                                                       */
/* ------------------------------------------------------------------ */

static size_t dt_size(int d) { return (d == DT_F64 || d == DT_I64) ? 8 : 4; }

static val get(const tval *t, int64_t i) {
  val v;
  switch (t->dt) {
    case DT_F32: v.f = ((const float *)t->data)[i]; break;
    case DT_F64: v.f = ((const double *)t->data)[i]; break;
    case DT_I32: v.i = ((const int32_t *)t->data)[i]; break;
    default: v.i = ((const int64_t *)t->data)[i]; break;
  }
  return v;
}

static void set(tval *t, int64_t i, val v) {
  switch (t->dt) {
    case DT_F32: ((float *)t->data)[i] = (float)v.f; break;
    case DT_F64: ((double *)t->data)[i] = v.f; break;
    case DT_I32: ((int32_t *)t->data)[i] = (int32_t)v.i; break;
    default: ((int64_t *)t->data)[i] = v.i; break;
  }
}

static void tval_new(tval *t, int dt, int rank, const int64_t *dims) {
  if (dt == DT_BOOL) fail("Value.create: Bool tensors are not storable");
  t->dt = dt;
  t->rank = rank;
  t->n = 1;
  for (int i = 0; i < rank; i++) {
    t->dims[i] = dims[i];
    t->n *= dims[i];
  }
  t->data = xcalloc((size_t)t->n, dt_size(dt));
  t->owned = 1;
}

static const char *DT_NAME[] = {"f32", "f64", "i32", "i64", "bool"};

static void shape_str(char *buf, size_t n, int rank, const int64_t *dims) {
  size_t k = (size_t)snprintf(buf, n, "[");
  for (int i = 0; i < rank && k < n; i++) k += (size_t)snprintf(buf + k, n - k, i ? ",%lld" : "%lld", (long long)dims[i]);
  if (k < n) snprintf(buf + k, n - k, "]");
}

static int64_t row_len(int rank, const int64_t *dims) { return rank ? dims[rank - 1] : 1; }

typedef struct {
  int n;
  const char *const *names;
  const int *dtypes;
  const int *ranks;
  const int64_t *const *dims;
  const void *const *data;
} inputs_t;

static void compute(const orc_graph *g, int p, tval *vals, const inputs_t *in, evalctx *c) {
  const tnode *t = &g->ts[p];
  tval *out = &vals[p];
  switch (t->kind) {
    case T_PARAM: {
      int k;
      for (k = 0; k < in->n; k++)
        if (strcmp(in->names[k], t->pname) == 0) break;
      if (k == in->n) fail("Backend_interp: missing input \"%s\"", t->pname);
      if (in->dtypes[k] != t->dt)
        fail("Backend_interp: input \"%s\" has dtype %s, expected %s", t->pname, DT_NAME[in->dtypes[k]], DT_NAME[t->dt]);
      int same = in->ranks[k] == t->rank;
      for (int d = 0; same && d < t->rank; d++) same = in->dims[k][d] == t->dims[d];
      if (!same) {
        char a[256], b[256];
        shape_str(a, sizeof a, in->ranks[k], in->dims[k]);
        shape_str(b, sizeof b, t->rank, t->dims);
        fail("Backend_interp: input \"%s\" has shape %s, expected %s", t->pname, a, b);
      }
      out->dt = t->dt;
      out->rank = t->rank;
      memcpy(out->dims, t->dims, sizeof t->dims);
      out->n = t->numel;
      out->data = (void *)in->data[k];
      out->owned = 0;
      return;
    }
    case T_IOTA:
      tval_new(out, DT_I32, t->rank, t->dims);
      for (int64_t i = 0; i < out->n; i++) ((int32_t *)out->data)[i] = (int32_t)i;
      return;
    case T_MAP: {
      const tval *s = &vals[t->a];
      tval_new(out, t->dt, t->rank, t->dims);
      c->nenv = 1;
      c->envdt[0] = s->dt;
      for (int64_t i = 0; i < out->n; i++) {
        c->env[0] = get(s, i);
        set(out, i, eval_at(c, t->body, i));
      }
      return;
    }
    case T_MAP2: {
      const tval *a = &vals[t->a], *b = &vals[t->b];
      tval_new(out, t->dt, t->rank, t->dims);
      c->nenv = 2;
      c->envdt[0] = a->dt;
      c->envdt[1] = b->dt;
      for (int64_t i = 0; i < out->n; i++) {
        c->env[0] = get(a, i);
        c->env[1] = get(b, i);
        set(out, i, eval_at(c, t->body, i));
      }
      return;
    }
    case T_REDUCE: {
      const tval *s = &vals[t->a];
      int64_t n = row_len(s->rank, s->dims);
      tval_new(out, t->dt, t->rank, t->dims);
      int64_t rows = out->n;
      for (int64_t r = 0; r < rows; r++) {
        c->nenv = 0;
        val acc = eval_at(c, t->init, 0);
        c->nenv = 2;
        c->envdt[0] = s->dt;
        c->envdt[1] = s->dt;
        for (int64_t j = 0; j < n; j++) {
          int64_t i = r * n + j;
          c->env[0] = acc;
          c->env[1] = get(s, i);
          acc = eval_at(c, t->body, i);
        }
        set(out, r, acc);
      }
      return;
    }
    case T_SCAN: {
      const tval *s = &vals[t->a];
      tval_new(out, t->dt, t->rank, t->dims);
      int64_t n = row_len(s->rank, s->dims);
      int64_t rows = n == 0 ? 0 : s->n / n;
      for (int64_t r = 0; r < rows; r++) {
        c->nenv = 0;
        val acc = eval_at(c, t->init, 0);
        c->nenv = 2;
        c->envdt[0] = s->dt;
        c->envdt[1] = s->dt;
        for (int64_t j = 0; j < n; j++) {
          int64_t i = r * n + j;
          c->env[0] = acc;
          c->env[1] = get(s, i);
          acc = eval_at(c, t->body, i);
          set(out, i, acc);
        }
      }
      return;
    }
    case T_GATHER: {
      const tval *ix = &vals[t->a], *s = &vals[t->b];
      tval_new(out, t->dt, t->rank, t->dims);
      for (int64_t i = 0; i < out->n; i++) {
        int64_t j = ((const int32_t *)ix->data)[i];
        if (j < 0 || j >= s->n)
          fail("Backend_interp: gather index out of bounds: %lld at %lld (source has %lld elements)", (long long)j,
               (long long)i, (long long)s->n);
        set(out, i, get(s, j));
      }
      return;
    }
    case T_SCATTER: {
      const tval *ix = &vals[t->a], *s = &vals[t->b];
      tval_new(out, t->dt, t->rank, t->dims);
      int64_t m = out->n;
      for (int64_t i = 0; i < s->n; i++) {
        int64_t j = ((const int32_t *)ix->data)[i];
        if (j < 0 || j >= m)
          fail("Backend_interp: scatter_add index out of bounds: %lld at %lld (output has %lld elements)", (long long)j,
               (long long)i, (long long)m);
        val o = get(out, j), v = get(s, i), r;
        switch (t->dt) {
          case DT_F32: r.f = round_f32(o.f + v.f); break;
          case DT_F64: r.f = o.f + v.f; break;
          case DT_I32: r.i = i32_binop(B_ADD, (int32_t)o.i, (int32_t)v.i); break;
          default: r.i = i64_binop(B_ADD, o.i, v.i); break;
        }
        set(out, j, r);
      }
      return;
    }
    case T_MATMUL: {
      const tval *a = &vals[t->a], *b = &vals[t->b];
      int64_t k = row_len(a->rank, a->dims);
      int64_t n = row_len(t->rank, t->dims);
      tval_new(out, t->dt, t->rank, t->dims);
      int64_t rows = n == 0 ? 0 : out->n / n;
      /* Built with -ffp-contract=off: the product is rounded, then the sum,
         exactly round_f32(acc + round_f32(a*b)) since a double holds any
         f32 product exactly and f32 + f32 rounds once either way. */
      if (t->dt == DT_F32) {
        const float *A = (const float *)a->data, *B = (const float *)b->data;
        float *O = (float *)out->data;
        for (int64_t i = 0; i < rows; i++)
          for (int64_t j = 0; j < n; j++) {
            float acc = 0.0f;
            for (int64_t p2 = 0; p2 < k; p2++) acc = acc + A[i * k + p2] * B[p2 * n + j];
            O[i * n + j] = acc;
          }
      } else if (t->dt == DT_F64) {
        const double *A = (const double *)a->data, *B = (const double *)b->data;
        double *O = (double *)out->data;
        for (int64_t i = 0; i < rows; i++)
          for (int64_t j = 0; j < n; j++) {
            double acc = 0.0;
            for (int64_t p2 = 0; p2 < k; p2++) acc = acc + A[i * k + p2] * B[p2 * n + j];
            O[i * n + j] = acc;
          }
      } else {
        for (int64_t i = 0; i < rows; i++)
          for (int64_t j = 0; j < n; j++) {
            val acc;
            acc.i = 0;
            for (int64_t p2 = 0; p2 < k; p2++) {
              val x = get(a, i * k + p2), y = get(b, p2 * n + j);
              if (t->dt == DT_I32)
                acc.i = i32_binop(B_ADD, (int32_t)acc.i, i32_binop(B_MUL, (int32_t)x.i, (int32_t)y.i));
              else
                acc.i = i64_binop(B_ADD, acc.i, i64_binop(B_MUL, x.i, y.i));
            }
            set(out, i * n + j, acc);
          }
      }
      return;
    }
    case T_RESHAPE: {
      const tval *s = &vals[t->a];
      tval_new(out, t->dt, t->rank, t->dims);
      memcpy(out->data, s->data, (size_t)out->n * dt_size(t->dt));
      return;
    }
    default: { /* broadcast */
      const tval *s = &vals[t->a];
      tval_new(out, t->dt, t->rank, t->dims);
      val x = get(s, 0);
      for (int64_t i = 0; i < out->n; i++) set(out, i, x);
      return;
    }
  }
}

void orc_result_free(orc_result *r) {
  if (!r) return;
  for (int i = 0; i < r->count; i++) {
    free(r->names[i]);
    if (r->vals[i].owned) free(r->vals[i].data);
  }
  free(r->names);
  free(r->vals);
  free(r);
}

orc_result *orc_run(const orc_graph *g, int nin, const char *const *names, const int *dtypes, const int *ranks,
                    const int64_t *const *dims, const void *const *data, char *err, int errlen) {
  jmp_buf jb;
  jmp_buf *saved = err_jmp;
  tval *volatile vals = NULL;
  int *volatile uses = NULL;
  orc_result *volatile res = NULL;
  evalctx c;
  memset(&c, 0, sizeof c);
  c.g = g;
  val *volatile memo = NULL;
  uint64_t *volatile stamp = NULL;
  err_jmp = &jb;
  if (setjmp(jb)) {
    err_jmp = saved;
    snprintf(err, (size_t)errlen, "%s", err_msg);
    if (vals)
      for (int i = 0; i < g->nt; i++)
        if (vals[i].owned) free(vals[i].data);
    free(vals);
    free(uses);
    free(memo);
    free(stamp);
    orc_result_free(res);
    return NULL;
  }
  inputs_t in = {nin, names, dtypes, ranks, dims, data};
  vals = (tval *)xcalloc((size_t)g->nt, sizeof(tval));
  uses = (int *)xcalloc((size_t)g->nt, sizeof(int));
  memo = (val *)xcalloc((size_t)(g->nx + 1), sizeof(val));
  stamp = (uint64_t *)xcalloc((size_t)(g->nx + 1), sizeof(uint64_t));
  c.memo = memo;
  c.stamp = stamp;
  for (int p = 0; p < g->nt; p++) {
    if (g->ts[p].a >= 0) uses[g->ts[p].a]++;
    if (g->ts[p].b >= 0) uses[g->ts[p].b]++;
  }
  for (int i = 0; i < g->no; i++) uses[g->otid[i]] += 1 << 20; /* outputs are never freed early */
  for (int p = 0; p < g->nt; p++) {
    compute(g, p, vals, &in, &c);
    int deps[2] = {g->ts[p].a, g->ts[p].b};
    for (int k = 0; k < 2; k++) {
      int d = deps[k];
      if (d < 0) continue;
      if (--uses[d] == 0 && vals[d].owned) {
        free(vals[d].data);
        vals[d].data = NULL;
        vals[d].owned = 0;
      }
    }
  }
  res = (orc_result *)xcalloc(1, sizeof(orc_result));
  res->names = (char **)xcalloc((size_t)g->no, sizeof(char *));
  res->vals = (tval *)xcalloc((size_t)g->no, sizeof(tval));
  res->count = g->no;
  for (int i = 0; i < g->no; i++) {
    res->names[i] = strdup(g->onames[i]);
    const tval *s = &vals[g->otid[i]];
    tval *d = &res->vals[i];
    d->dt = s->dt;
    d->rank = g->ts[g->otid[i]].rank;
    memcpy(d->dims, g->ts[g->otid[i]].dims, sizeof d->dims);
    d->n = s->n;
    d->data = xmalloc((size_t)s->n * dt_size(s->dt));
    memcpy(d->data, s->data, (size_t)s->n * dt_size(s->dt));
    d->owned = 1;
  }
  for (int p = 0; p < g->nt; p++)
    if (vals[p].owned) free(vals[p].data);
  free(vals);
  free(uses);
  free(memo);
  free(stamp);
  err_jmp = saved;
  return res;
}

int orc_result_count(const orc_result *r) { return r->count; }
const char *orc_result_name(const orc_result *r, int i) { return r->names[i]; }
int orc_result_dtype(const orc_result *r, int i) { return r->vals[i].dt; }
int orc_result_rank(const orc_result *r, int i) { return r->vals[i].rank; }
const int64_t *orc_result_dims(const orc_result *r, int i) { return r->vals[i].dims; }
const void *orc_result_data(const orc_result *r, int i) { return r->vals[i].data; }

/* Philox-4x32-10 on the host, one block: the generator the synthetic
   inputs are drawn from. Written from the published algorithm (Salmon et
   al., SC'11) with Random123's round constants; pinned by the Random123
   known-answer vectors in the tests. */
void orc_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
  uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
  uint32_t k0 = key_in[0], k1 = key_in[1];
  for (int r = 0; r < 10; r++) {
    uint64_t p0 = (uint64_t)0xD2511F53u * c0;
    uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
    uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
    uint32_t n1 = (uint32_t)p1;
    uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
    uint32_t n3 = (uint32_t)p0;
    c0 = n0;
    c1 = n1;
    c2 = n2;
    c3 = n3;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  out[0] = c0;
  out[1] = c1;
  out[2] = c2;
  out[3] = c3;
}
