// Shared declarations of the cchip library: error plumbing, the graph model
// the wire parser builds, the fusion plan, and the program description the
// code generator hands to the executor.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace cchip {

// ---------------------------------------------------------------------------
// Errors: Invalid_argument and Failure of the reference, as exceptions that
// the C-ABI layer turns into status codes.
// ---------------------------------------------------------------------------

struct InvalidArgument : std::runtime_error {
  using std::runtime_error::runtime_error;
};
struct Failure : std::runtime_error {
  using std::runtime_error::runtime_error;
};

std::string strf(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
void set_last_error(const std::string &msg);

template <typename F>
int guarded(F &&f) {
  try {
    f();
    return 0;
  } catch (const InvalidArgument &e) {
    set_last_error(e.what());
    return 1;
  } catch (const Failure &e) {
    set_last_error(e.what());
    return 2;
  } catch (const std::exception &e) {
    set_last_error(e.what());
    return 2;
  }
}

// ---------------------------------------------------------------------------
// Dtypes (lib/ir/dtype.ml:9-46)
// ---------------------------------------------------------------------------

enum class DT : int { F32 = 0, F64 = 1, I32 = 2, I64 = 3, BOOL = 4 };

inline int dt_size(DT d) { return (d == DT::F64 || d == DT::I64) ? 8 : (d == DT::BOOL ? 1 : 4); }
inline bool dt_is_float(DT d) { return d == DT::F32 || d == DT::F64; }
const char *dt_name(DT d);
const char *dt_ctype(DT d);

// ---------------------------------------------------------------------------
// Graph model (lib/ir/expr.ml, lib/ir/tensor.ml, lib/ir/graph.ml)
// ---------------------------------------------------------------------------

enum class XK { Const, Arg, Index, Bin, Un, Cmp, Logic, Not, Select, Cast };
enum Bin { B_ADD, B_SUB, B_MUL, B_DIV, B_MIN, B_MAX, B_AND, B_OR, B_XOR, B_SHL, B_SHR };
enum Un { U_NEG, U_SQRT, U_EXP, U_LOG, U_ABS, U_SIN, U_COS, U_ERF, U_ERFINV };
enum Cmp { C_EQ, C_NE, C_LT, C_LE, C_GT, C_GE };

struct XNode {
  int64_t id = 0;
  XK kind = XK::Const;
  DT dt = DT::F32;
  int op = 0;
  int a = -1, b = -1, c = -1;  // positions
  double f = 0;                 // float constant, the double as written
  int64_t i = 0;                // integer / bool constant
  int arg = 0;
};

enum class TK { Param, Iota, Map, Map2, Reduce, Scan, Gather, Scatter, Matmul, Reshape, Broadcast };

struct TNode {
  int64_t id = 0;
  TK kind = TK::Param;
  DT dt = DT::F32;
  std::vector<int64_t> shape;
  int64_t numel = 1;
  int a = -1, b = -1;           // operand positions
  int init = -1, body = -1;     // expression positions
  std::string pname;
  std::vector<int> deps() const {
    std::vector<int> d;
    if (a >= 0) d.push_back(a);
    if (b >= 0) d.push_back(b);
    return d;
  }
};

struct Graph {
  std::string name;
  std::vector<XNode> xs;
  std::vector<TNode> ts;  // topological order
  std::vector<std::pair<std::string, int>> outputs;
  std::vector<int> fan_out;  // uses per tensor position
};

Graph parse_wire(const std::string &text);
int64_t row_length(const std::vector<int64_t> &shape);

// Fusion.plan (lib/lower/fusion.ml:41-73): a node owns a buffer iff it is a
// Param, a barrier (Reduce, Scan, Scatter_add, Matmul), an output, or has
// fan-out >= 2. Roots are the materialised non-params in topological order.
struct Plan {
  std::vector<bool> materialized;
  std::vector<int> roots;
};
Plan fusion_plan(const Graph &g);

// Position of x if tensor t is Dsl.transpose x (a gather whose index is the
// transpose map over iota), else -1.
int transpose_source(const Graph &g, int t);

// ---------------------------------------------------------------------------
// Program: what the code generator produces and the executor runs
// (Kernel_ir.program, lib/lower/kernel_ir.ml:124-141).
// ---------------------------------------------------------------------------

enum class BufRole { Param, Computed, Scratch, Err };

struct BufSpec {
  std::string name;
  DT dt = DT::F32;
  int64_t numel = 0;
  BufRole role = BufRole::Computed;
  // A materialised tensor that no kernel reads and the graph does not
  // output (a broadcast its consumers recompute): never allocated, its
  // kernel not launched.
  bool elided = false;
  int64_t bytes() const { return numel * dt_size(dt); }
};

struct KernelSpec {
  std::string name;
  std::vector<int> args;  // buffer indices, in parameter order
  int grid = 1, grid_y = 1, block = 256, block_y = 1, shared_bytes = 0;
  std::string role;       // template that produced it, for the plan dump
  // Algorithmic bytes of the root this kernel computes (each element the
  // root reads counted once, its output written once), on the root's main
  // kernel; 0 on helper kernels (look-back init, scatter bookkeeping, ...).
  int64_t algo_bytes = 0;
  // Bytes the kernel itself reads from and writes to materialised tensors
  // (scratch excluded), each tensor read once: the root's algorithmic
  // bytes, less reads the lowering made unnecessary (a reduction folded
  // inside the map that writes its input reads nothing back; roots over
  // one input fused into one kernel read it once). 0 on helper kernels.
  int64_t moved_bytes = 0;
};

enum class OpK { Alloc, Upload, Launch, Download, Free };

struct HostOp {
  OpK kind;
  int buf = -1;       // Alloc/Upload/Download/Free
  int kernel = -1;    // Launch
  std::string name;   // Upload: param; Download: output
};

struct IOSpec {
  std::string name;
  DT dt;
  std::vector<int64_t> shape;
  int buf;
};

struct ProgramIR {
  std::string name;
  std::string source;
  std::vector<BufSpec> bufs;
  std::vector<KernelSpec> kernels;
  std::vector<HostOp> plan;
  std::vector<IOSpec> params;
  std::vector<IOSpec> outputs;
  int err_buf = -1;
};

ProgramIR lower_program(const Graph &g);
std::string plan_to_string(const ProgramIR &p);
// A CCHIP_TUNE knob ("key=value,..."), or dflt when unset.
int64_t tune_knob(const char *key, int64_t dflt);

// ---------------------------------------------------------------------------
// Runtime internals shared with the executor
// ---------------------------------------------------------------------------

void check_hip(int status, const char *what);
void ensure_init();
void *rt_alloc(size_t bytes);
void rt_free(void *p);

struct Module;
std::shared_ptr<Module> jit_compile(const std::string &name, const std::string &source);
void *module_kernel(Module &m, const std::string &name);
std::vector<char> jit_code_object(const std::string &name, const std::string &source);

// The static scratch of the allocation-free entry point (noalloc.hip).
size_t noalloc_scratch_capacity();
void *noalloc_scratch(int device);
void noalloc_scratch_clear(void *base, size_t bytes, void *stream);

}  // namespace cchip
