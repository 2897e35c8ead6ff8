// Backend_hip: compile (plan + templates + JIT + pools) and the executor
// that walks the host plan, behind the C ABI of include/cchip_backend.h.
//
// Restates lib/backend_cuda/executor.ml:23-244 and
// lib/backend_cuda/cudacaml_backend_cuda.ml:23-111 on HIP: a compiled
// program owns `streams` executors, each with its own stream and buffer
// pool allocated once at compile time; a run only uploads, launches and
// downloads, all ordered by the executor's stream; run_resident substitutes
// the caller's device buffers for the plan's own by name.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <mutex>

#include "../../include/cchip_backend.h"
#include "internal.hpp"

using namespace cchip;

namespace {

struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    ensure_init();
    check_hip(hipGetDevice(&prev), "hipGetDevice");
    if (prev != dev) check_hip(hipSetDevice(dev), "hipSetDevice");
  }
  ~DeviceGuard() {
    int cur = -1;
    if (hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

// A recorded launch sequence for one set of buffer pointers.
struct GraphEntry {
  std::vector<void *> key;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

struct Executor {
  hipStream_t stream = nullptr;
  // Launch sequences are recorded on this private stream (lane 0 runs on
  // the null stream, which cannot be captured) and replayed on `stream`;
  // most recently used last.
  hipStream_t capture = nullptr;
  std::vector<GraphEntry> graphs;
  std::vector<void *> bufs;
  int *err_host = nullptr;  // pinned word the error flag is read into
  // Small params, the error word and small outputs share one device
  // allocation, mirrored by one pinned host block: a synchronous run moves
  // them with one copy each way instead of one pageable copy (and, for a
  // download, one round trip to the device) per value. Layout: the params
  // in [0, arena_in), then the error word and the outputs.
  char *arena = nullptr;
  char *arena_host = nullptr;
  size_t arena_in = 0, arena_bytes = 0;
  std::vector<int64_t> off;  // per buffer: its offset in the arena, or -1
};

// Recorded launch sequences kept per executor (distinct pointer sets).
constexpr size_t kGraphCache = 8;

// A value of at most this many bytes travels through the arena.
constexpr size_t kArenaValue = 4096;
constexpr size_t kArenaMax = size_t(1) << 20;

const char *err_message(int code) {
  if (code & 1) return "Backend_hip: gather index out of bounds";
  if (code & 2) return "Backend_hip: scatter_add index out of bounds";
  return "Backend_hip: scan look-back did not complete (device-side timeout)";
}

}  // namespace

struct cchip_program {
  ProgramIR ir;
  std::shared_ptr<Module> mod;
  std::vector<void *> kfn;
  int device = 0;
  std::vector<Executor> execs;
  int next = 0;
  bool released = false;
  bool graphs = false;  // replay launch sequences as HIP graphs
  std::mutex mu;
  // timing hook
  int timed = -1;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> ev_used, ev_free;
  // Allocation-free runs (cchip_program_run_resident_noalloc): each scratch
  // buffer's offset in the static scratch (-1 for other buffers) and their
  // total, which outputs are copied rather than written in place, and host
  // arrays sized here so that such a run allocates no memory at all.
  std::vector<int64_t> na_off;
  int64_t na_bytes = 0;
  std::vector<char> na_out_copy;
  std::vector<int> na_which;
  std::vector<void *> na_ptr, na_vals, na_args;
};

struct cchip_job {
  cchip_program *prog = nullptr;
  int lane = 0;
  hipEvent_t done = nullptr;
  // The job's own pinned copy of the device error word, written by its
  // lane's stream at the end of the job's work: jobs queued on one lane
  // never see each other's flags.
  int *err = nullptr;
  bool waited = false;
  int status = 0;
  std::string msg;
};

namespace {

// Pinned error slots of asynchronous jobs, shared by every program of the
// process and recycled when a job is freed (a job may outlive its
// program). Allocated in blocks, never returned to the driver.
std::mutex g_slot_mu;
std::vector<int *> g_slot_free;
constexpr int kSlotBlock = 256;

int *err_slot_get() {
  std::lock_guard<std::mutex> lk(g_slot_mu);
  if (g_slot_free.empty()) {
    int *blk = nullptr;
    check_hip(hipHostMalloc((void **)&blk, kSlotBlock * sizeof(int), hipHostMallocPortable), "hipHostMalloc");
    for (int i = kSlotBlock - 1; i >= 0; i--) g_slot_free.push_back(blk + i);
  }
  int *s = g_slot_free.back();
  g_slot_free.pop_back();
  *s = 0;
  return s;
}

void err_slot_put(int *s) {
  if (!s) return;
  std::lock_guard<std::mutex> lk(g_slot_mu);
  g_slot_free.push_back(s);
}

void release_program(cchip_program *p) {
  if (p->released) return;
  p->released = true;
  DeviceGuard dg(p->device);
  for (auto &e : p->execs) {
    if (e.stream) (void)hipStreamSynchronize(e.stream);
    else (void)hipDeviceSynchronize();
    for (auto &g : e.graphs) {
      if (g.exec) (void)hipGraphExecDestroy(g.exec);
      if (g.graph) (void)hipGraphDestroy(g.graph);
    }
    e.graphs.clear();
    if (e.capture) (void)hipStreamDestroy(e.capture);
    e.capture = nullptr;
    for (size_t b = 0; b < e.bufs.size(); b++)
      if (e.off.empty() || e.off[b] < 0) rt_free(e.bufs[b]);
    e.bufs.clear();
    if (e.arena) rt_free(e.arena);
    if (e.arena_host) (void)hipHostFree(e.arena_host);
    e.arena = e.arena_host = nullptr;
    if (e.err_host) (void)hipHostFree(e.err_host);
    e.err_host = nullptr;
    if (e.stream) (void)hipStreamDestroy(e.stream);
    e.stream = nullptr;
  }
  for (auto &pr : p->ev_used) {
    (void)hipEventDestroy(pr.first);
    (void)hipEventDestroy(pr.second);
  }
  for (auto &pr : p->ev_free) {
    (void)hipEventDestroy(pr.first);
    (void)hipEventDestroy(pr.second);
  }
  p->ev_used.clear();
  p->ev_free.clear();
  p->mod.reset();
}

const IOSpec *find_param(const ProgramIR &ir, const std::string &name) {
  for (auto &p : ir.params)
    if (p.name == name) return &p;
  return nullptr;
}

// Every input must be present, with the param's exact byte size, before any
// device work is issued (executor.ml:12-21, :192-208).
std::vector<int> bind_inputs(const cchip_program *p, int n, const char *const *names, const size_t *bytes,
                             const char *who) {
  std::vector<int> which(p->ir.params.size(), -1);
  for (size_t k = 0; k < p->ir.params.size(); k++) {
    const IOSpec &ps = p->ir.params[k];
    for (int i = 0; i < n; i++)
      if (names[i] && ps.name == names[i]) {
        which[k] = i;
        break;
      }
    if (which[k] < 0) throw InvalidArgument(std::string(who) + ": missing input " + ps.name);
    size_t want = (size_t)p->ir.bufs[ps.buf].bytes();
    if (bytes[which[k]] != want)
      throw InvalidArgument(strf("%s: input %s is %zu bytes, parameter %s needs %zu", who, ps.name.c_str(),
                                 bytes[which[k]], p->ir.bufs[ps.buf].name.c_str(), want));
  }
  return which;
}

void issue_launches(cchip_program *p, hipStream_t stream, const std::vector<void *> &ptr, bool timing) {
  for (auto &op : p->ir.plan) {
    if (op.kind != OpK::Launch) continue;
    const KernelSpec &k = p->ir.kernels[op.kernel];
    std::vector<void *> vals(k.args.size());
    std::vector<void *> args(k.args.size());
    for (size_t i = 0; i < k.args.size(); i++) {
      vals[i] = ptr[k.args[i]];
      args[i] = &vals[i];
    }
    bool timed = timing && op.kernel == p->timed;
    std::pair<hipEvent_t, hipEvent_t> ev{nullptr, nullptr};
    if (timed) {
      if (!p->ev_free.empty()) {
        ev = p->ev_free.back();
        p->ev_free.pop_back();
      } else {
        check_hip(hipEventCreate(&ev.first), "hipEventCreate");
        check_hip(hipEventCreate(&ev.second), "hipEventCreate");
      }
      check_hip(hipEventRecord(ev.first, stream), "hipEventRecord");
    }
    check_hip(hipModuleLaunchKernel((hipFunction_t)p->kfn[op.kernel], k.grid, k.grid_y, 1, k.block, k.block_y, 1,
                                    k.shared_bytes, stream, args.data(), nullptr),
              "hipModuleLaunchKernel");
    if (timed) {
      check_hip(hipEventRecord(ev.second, stream), "hipEventRecord");
      p->ev_used.push_back(ev);
    }
  }
}

// The plan's launches on the executor's stream: replayed from a recorded
// HIP graph when graphs are on (CCHIP_TUNE graphs=1), the program has
// several kernels and none is being timed (one graph launch in place of a
// launch call per kernel), else issued one by one. Graphs are recorded per set of buffer pointers, since the
// kernels' arguments are baked into them.
void launch_kernels(cchip_program *p, Executor &e, const std::vector<void *> &ptr, bool timing) {
  if (!p->graphs || (timing && p->timed >= 0)) {
    issue_launches(p, e.stream, ptr, timing);
    return;
  }
  for (size_t i = 0; i < e.graphs.size(); i++)
    if (e.graphs[i].key == ptr) {
      std::rotate(e.graphs.begin() + i, e.graphs.begin() + i + 1, e.graphs.end());
      check_hip(hipGraphLaunch(e.graphs.back().exec, e.stream), "hipGraphLaunch");
      return;
    }
  if (!e.capture) check_hip(hipStreamCreateWithFlags(&e.capture, hipStreamNonBlocking), "hipStreamCreateWithFlags");
  GraphEntry g;
  g.key = ptr;
  check_hip(hipStreamBeginCapture(e.capture, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
  try {
    issue_launches(p, e.capture, ptr, false);
  } catch (...) {
    hipGraph_t partial = nullptr;
    (void)hipStreamEndCapture(e.capture, &partial);
    if (partial) (void)hipGraphDestroy(partial);
    throw;
  }
  check_hip(hipStreamEndCapture(e.capture, &g.graph), "hipStreamEndCapture");
  hipError_t rc = hipGraphInstantiate(&g.exec, g.graph, nullptr, nullptr, 0);
  if (rc != hipSuccess) {
    (void)hipGraphDestroy(g.graph);
    check_hip(rc, "hipGraphInstantiate");
  }
  if (e.graphs.size() >= kGraphCache) {
    (void)hipGraphExecDestroy(e.graphs.front().exec);
    (void)hipGraphDestroy(e.graphs.front().graph);
    e.graphs.erase(e.graphs.begin());
  }
  e.graphs.push_back(g);
  check_hip(hipGraphLaunch(e.graphs.back().exec, e.stream), "hipGraphLaunch");
}

// The device error word is sticky: kernels only ever set bits in it. A run
// that reports errors queues, on its own stream and after its kernels, a
// copy of the word into a host slot (the run's own: the pinned block of a
// synchronous run, the job's slot of an asynchronous one) and then a reset
// of the word. Runs on one lane are ordered by its stream, so each run
// reads exactly the flags of the runs since the previous read; lanes have
// separate words.
void queue_err_reset(cchip_program *p, Executor &e) {
  if (p->ir.err_buf < 0) return;
  check_hip(hipMemsetAsync(e.bufs[p->ir.err_buf], 0, sizeof(int), e.stream), "hipMemsetAsync err");
}

void queue_err_read(cchip_program *p, Executor &e, int *slot) {
  if (p->ir.err_buf < 0) return;
  check_hip(hipMemcpyAsync(slot, e.bufs[p->ir.err_buf], sizeof(int), hipMemcpyDeviceToHost, e.stream),
            "hipMemcpyAsync err");
  queue_err_reset(p, e);
}

// A run that failed after some of its work was queued: wait for that work,
// then clear the lane's error word, so that flags its kernels may have set
// are not reported by the next run on the lane.
void discard_err(cchip_program *p, Executor &e) {
  (void)hipStreamSynchronize(e.stream);
  if (p->ir.err_buf < 0 || p->ir.err_buf >= (int)e.bufs.size()) return;
  if (hipMemsetAsync(e.bufs[p->ir.err_buf], 0, sizeof(int), e.stream) == hipSuccess)
    (void)hipStreamSynchronize(e.stream);
}

// After the run's stream has been waited on: raise the interpreter's error
// for the flags its slot received.
void raise_err_slot(cchip_program *p, int *slot) {
  if (p->ir.err_buf < 0 || !slot) return;
  int code = *slot;
  *slot = 0;
  if (code) throw InvalidArgument(err_message(code));
}

// Issues a run from host memory. With `staged` (the synchronous run, which
// waits before it returns) the arena's values go through its pinned block;
// the caller copies the small outputs out after the wait (finish_staged).
// Asynchronous runs copy straight between the caller's memory and the
// device, since several may be in flight on one lane.
void issue_host_run(cchip_program *p, int lane, int n, const char *const *names, const void *const *host,
                    const size_t *bytes, void *const *outputs, bool staged, int *err_slot) {
  if (p->released) throw Failure("Executor.run: this executor has been released");
  std::vector<int> which = bind_inputs(p, n, names, bytes, "Executor.run");
  Executor &e = p->execs[lane];
  staged = staged && e.arena;
  const std::vector<void *> &ptr = e.bufs;
  for (size_t k = 0; k < p->ir.params.size(); k++) {
    const IOSpec &ps = p->ir.params[k];
    size_t nb = (size_t)p->ir.bufs[ps.buf].bytes();
    if (!nb) continue;
    if (staged && e.off[ps.buf] >= 0)
      memcpy(e.arena_host + e.off[ps.buf], host[which[k]], nb);
    else
      check_hip(hipMemcpyAsync(ptr[ps.buf], host[which[k]], nb, hipMemcpyHostToDevice, e.stream), "upload");
  }
  if (staged && e.arena_in)
    check_hip(hipMemcpyAsync(e.arena, e.arena_host, e.arena_in, hipMemcpyHostToDevice, e.stream), "upload");
  launch_kernels(p, e, ptr, lane == 0);
  for (size_t o = 0; o < p->ir.outputs.size(); o++) {
    const IOSpec &os = p->ir.outputs[o];
    size_t nb = (size_t)p->ir.bufs[os.buf].bytes();
    if (!nb || (staged && e.off[os.buf] >= 0)) continue;
    check_hip(hipMemcpyAsync(outputs[o], ptr[os.buf], nb, hipMemcpyDeviceToHost, e.stream), "download");
  }
  if (staged) {
    if (e.arena_bytes > e.arena_in)
      check_hip(hipMemcpyAsync(e.arena_host + e.arena_in, e.arena + e.arena_in, e.arena_bytes - e.arena_in,
                               hipMemcpyDeviceToHost, e.stream),
                "download");
    // the error word travelled with the block when it lives there
    if (p->ir.err_buf >= 0 && e.off[p->ir.err_buf] >= 0) queue_err_reset(p, e);
    else queue_err_read(p, e, err_slot);
  } else {
    queue_err_read(p, e, err_slot);
  }
}

// After the wait of a staged run: raise the device's error, if any, and
// copy the small outputs out of the pinned block.
void finish_staged(cchip_program *p, Executor &e, void *const *outputs) {
  if (p->ir.err_buf >= 0) {
    const int64_t at = e.off[p->ir.err_buf];
    raise_err_slot(p, at >= 0 ? (int *)(e.arena_host + at) : e.err_host);
  }
  if (!e.arena) return;
  for (size_t o = 0; o < p->ir.outputs.size(); o++) {
    const IOSpec &os = p->ir.outputs[o];
    size_t nb = (size_t)p->ir.bufs[os.buf].bytes();
    if (nb && e.off[os.buf] >= 0) memcpy(outputs[o], e.arena_host + e.off[os.buf], nb);
  }
}

void run_resident_impl(cchip_program *p, int n, const char *const *names, void *const *dev_inputs,
                       const size_t *bytes, void **outs_alloc, void *const *outs_given, bool sync) {
  if (p->released) throw Failure("Executor.run_resident: this executor has been released");
  std::vector<int> which = bind_inputs(p, n, names, bytes, "Executor.run_resident");
  Executor &e = p->execs[0];
  std::vector<void *> ptr = e.bufs;
  std::vector<bool> overridden(ptr.size(), false);
  for (size_t k = 0; k < p->ir.params.size(); k++) {
    ptr[p->ir.params[k].buf] = dev_inputs[which[k]];
    overridden[p->ir.params[k].buf] = true;
  }
  // Outputs: substitute a fresh (or caller-given) buffer for the plan's own
  // so the producing kernel writes straight into it; a name already bound
  // (an output that is a param, or one buffer downloaded twice) is copied.
  std::vector<std::pair<int, void *>> copies;
  std::vector<void *> fresh;
  try {
    for (size_t o = 0; o < p->ir.outputs.size(); o++) {
      const IOSpec &os = p->ir.outputs[o];
      void *dst;
      if (outs_given) {
        dst = outs_given[o];
      } else {
        dst = rt_alloc((size_t)p->ir.bufs[os.buf].bytes());
        fresh.push_back(dst);
      }
      if (overridden[os.buf]) copies.emplace_back(os.buf, dst);
      else {
        ptr[os.buf] = dst;
        overridden[os.buf] = true;
      }
      if (outs_alloc) outs_alloc[o] = dst;
    }
    launch_kernels(p, e, ptr, true);
    for (auto &c : copies) {
      size_t nb = (size_t)p->ir.bufs[c.first].bytes();
      if (nb) check_hip(hipMemcpyAsync(c.second, ptr[c.first], nb, hipMemcpyDeviceToDevice, e.stream), "copy_device");
    }
    if (sync) {
      queue_err_read(p, e, e.err_host);
      check_hip(hipStreamSynchronize(e.stream), "hipStreamSynchronize");
      raise_err_slot(p, e.err_host);
    }
  } catch (...) {
    if (sync) discard_err(p, e);
    for (void *f : fresh) rt_free(f);
    throw;
  }
}

// Host-side layout of an allocation-free run, fixed at compile time: the
// call's own error word in the first 256 bytes of the static scratch (every
// program has the slot, so a caller's err_out always receives a defined
// word), then the scratch buffers packed 256-byte aligned, in buffer order
// (all of them at once, as the pool holds them).
void prepare_noalloc(cchip_program *p) {
  const ProgramIR &ir = p->ir;
  p->na_off.assign(ir.bufs.size(), -1);
  if (ir.err_buf >= 0) p->na_off[ir.err_buf] = 0;
  int64_t at = 256;
  for (size_t b = 0; b < ir.bufs.size(); b++)
    if (ir.bufs[b].role == BufRole::Scratch) {
      p->na_off[b] = at;
      at += (std::max<int64_t>(ir.bufs[b].bytes(), 1) + 255) & ~int64_t(255);
    }
  p->na_bytes = at;
  p->na_out_copy.assign(ir.outputs.size(), 0);
  std::vector<char> bound(ir.bufs.size(), 0);
  for (auto &ps : ir.params) bound[ps.buf] = 1;
  for (size_t o = 0; o < ir.outputs.size(); o++) {
    int b = ir.outputs[o].buf;
    if (bound[b]) p->na_out_copy[o] = 1;
    bound[b] = 1;
  }
  p->na_which.assign(ir.params.size(), -1);
  p->na_ptr.assign(ir.bufs.size(), nullptr);
  size_t maxargs = 1;
  for (auto &k : ir.kernels) maxargs = std::max(maxargs, k.args.size());
  p->na_vals.assign(maxargs, nullptr);
  p->na_args.assign(maxargs, nullptr);
  // the static scratch's address on this device (current here), looked up
  // now, at set-up; a failure surfaces on the first allocation-free run
  try {
    (void)noalloc_scratch(p->device);
  } catch (...) {
  }
}

}  // namespace

extern "C" {

void cchip_free(void *p) { free(p); }

static char *dup_string(const std::string &s) {
  char *c = (char *)malloc(s.size() + 1);
  memcpy(c, s.c_str(), s.size() + 1);
  return c;
}

int cchip_backend_source(const char *graph, char **source) {
  return guarded([&] {
    Graph g = parse_wire(graph);
    ProgramIR ir = lower_program(g);
    *source = dup_string(ir.source);
  });
}

int cchip_backend_plan(const char *graph, char **plan) {
  return guarded([&] {
    Graph g = parse_wire(graph);
    ProgramIR ir = lower_program(g);
    *plan = dup_string(plan_to_string(ir));
  });
}

int cchip_backend_compile(const char *graph, int device, int streams, cchip_program **program) {
  return guarded([&] {
    if (streams < 1) throw InvalidArgument("Backend_hip.compile_on: streams must be >= 1");
    Graph g = parse_wire(graph);
    auto p = std::make_unique<cchip_program>();
    p->ir = lower_program(g);
    p->device = device;
    ensure_init();
    int ndev = 0;
    check_hip(hipGetDeviceCount(&ndev), "hipGetDeviceCount");
    if (device < 0 || device >= ndev) throw InvalidArgument(strf("Backend_hip.compile_on: no device %d", device));
    DeviceGuard dg(device);
    p->mod = jit_compile("cchip_" + g.name, p->ir.source);
    int nlaunch = 0;
    for (auto &op : p->ir.plan) nlaunch += op.kind == OpK::Launch;
    // Off by default: on gfx950 a replayed graph measured no faster than
    // eager launches for resident steps, and slower for short host runs.
    p->graphs = tune_knob("graphs", 0) != 0 && nlaunch >= tune_knob("graph_min_kernels", 2);
    for (auto &k : p->ir.kernels) p->kfn.push_back(module_kernel(*p->mod, k.name));
    prepare_noalloc(p.get());
    p->execs.resize(streams);
    try {
      for (int s = 0; s < streams; s++) {
        Executor &e = p->execs[s];
        if (s > 0) check_hip(hipStreamCreateWithFlags(&e.stream, hipStreamNonBlocking), "hipStreamCreateWithFlags");
        check_hip(hipHostMalloc((void **)&e.err_host, sizeof(int), hipHostMallocPortable), "hipHostMalloc");
        *e.err_host = 0;
        e.bufs.assign(p->ir.bufs.size(), nullptr);
        e.off.assign(p->ir.bufs.size(), -1);
        size_t at = 0;
        auto place = [&](int b) {
          if (b < 0 || e.off[b] >= 0) return;
          size_t nb = (size_t)p->ir.bufs[b].bytes();
          size_t slot = (std::max<size_t>(nb, 1) + 255) & ~size_t(255);
          if (nb > kArenaValue || at + slot > kArenaMax) return;
          e.off[b] = (int64_t)at;
          at += slot;
        };
        for (auto &ps : p->ir.params) place(ps.buf);
        e.arena_in = at;
        if (p->ir.err_buf >= 0) place(p->ir.err_buf);
        for (auto &os : p->ir.outputs) place(os.buf);
        e.arena_bytes = at;
        if (at) {
          e.arena = (char *)rt_alloc(at);
          check_hip(hipMemset(e.arena, 0, at), "hipMemset");
          check_hip(hipHostMalloc((void **)&e.arena_host, at, hipHostMallocPortable), "hipHostMalloc");
          memset(e.arena_host, 0, at);
        }
        for (size_t b = 0; b < p->ir.bufs.size(); b++) {
          if (e.off[b] >= 0) {
            e.bufs[b] = e.arena + e.off[b];
            continue;
          }
          if (p->ir.bufs[b].elided) continue;  // no kernel reads or writes it
          e.bufs[b] = rt_alloc((size_t)p->ir.bufs[b].bytes());
          // Scratch (per-row counters, look-back status) and the error word
          // start at zero; the kernels leave them at zero again.
          if (p->ir.bufs[b].role == BufRole::Scratch || p->ir.bufs[b].role == BufRole::Err)
            check_hip(hipMemset(e.bufs[b], 0, (size_t)std::max<int64_t>(1, p->ir.bufs[b].bytes())), "hipMemset");
        }
      }
    } catch (...) {
      release_program(p.get());
      throw;
    }
    *program = p.release();
  });
}

int cchip_program_release(cchip_program *p) {
  return guarded([&] {
    if (!p) throw InvalidArgument("null program");
    std::lock_guard<std::mutex> lk(p->mu);
    release_program(p);
  });
}

int cchip_program_destroy(cchip_program *p) {
  int rc = cchip_program_release(p);
  delete p;
  return rc;
}

int cchip_program_device(const cchip_program *p) { return p->device; }
int cchip_program_streams(const cchip_program *p) { return (int)p->execs.size(); }
int cchip_program_buffer_count(const cchip_program *p) {
  if (p->released || p->execs.empty()) return 0;
  const Executor &e = p->execs[0];
  int n = e.arena ? 1 : 0;
  for (int64_t o : e.off) n += o < 0;
  return n;
}
int cchip_program_kernel_count(const cchip_program *p) { return (int)p->ir.kernels.size(); }
const char *cchip_program_kernel_name(const cchip_program *p, int i) {
  if (i < 0 || i >= (int)p->ir.kernels.size()) return nullptr;
  return p->ir.kernels[i].name.c_str();
}

static int io_info(const std::vector<IOSpec> &v, int i, const char **name, int *dtype, int *rank, int64_t *dims) {
  return guarded([&] {
    if (i < 0 || i >= (int)v.size()) throw InvalidArgument(strf("index %d out of range", i));
    const IOSpec &s = v[i];
    if (name) *name = s.name.c_str();
    if (dtype) *dtype = (int)s.dt;
    if (rank) *rank = (int)s.shape.size();
    if (dims)
      for (size_t k = 0; k < s.shape.size() && k < 8; k++) dims[k] = s.shape[k];
  });
}

int cchip_program_num_params(const cchip_program *p) { return (int)p->ir.params.size(); }
int cchip_program_param(const cchip_program *p, int i, const char **name, int *dtype, int *rank, int64_t *dims) {
  return io_info(p->ir.params, i, name, dtype, rank, dims);
}
int cchip_program_num_outputs(const cchip_program *p) { return (int)p->ir.outputs.size(); }
int cchip_program_output(const cchip_program *p, int i, const char **name, int *dtype, int *rank, int64_t *dims) {
  return io_info(p->ir.outputs, i, name, dtype, rank, dims);
}

int cchip_program_run(cchip_program *p, int n, const char *const *names, const void *const *host,
                      const size_t *bytes, void *const *outputs) {
  return guarded([&] {
    std::lock_guard<std::mutex> lk(p->mu);
    DeviceGuard dg(p->device);
    try {
      issue_host_run(p, 0, n, names, host, bytes, outputs, true, p->execs.empty() ? nullptr : p->execs[0].err_host);
      check_hip(hipStreamSynchronize(p->execs[0].stream), "hipStreamSynchronize");
    } catch (const InvalidArgument &) {
      throw;  // a caller mistake, found before any device work
    } catch (...) {
      if (!p->released && !p->execs.empty()) discard_err(p, p->execs[0]);
      throw;
    }
    finish_staged(p, p->execs[0], outputs);
  });
}

int cchip_program_run_async(cchip_program *p, int n, const char *const *names, const void *const *host,
                            const size_t *bytes, void *const *outputs, cchip_job **job) {
  return guarded([&] {
    std::lock_guard<std::mutex> lk(p->mu);
    DeviceGuard dg(p->device);
    int lane = p->next;
    auto j = std::make_unique<cchip_job>();
    j->prog = p;
    j->lane = lane;
    if (p->ir.err_buf >= 0) j->err = err_slot_get();
    try {
      issue_host_run(p, lane, n, names, host, bytes, outputs, false, j->err);
      check_hip(hipEventCreateWithFlags(&j->done, hipEventDisableTiming), "hipEventCreate");
      check_hip(hipEventRecord(j->done, p->execs[lane].stream), "hipEventRecord");
    } catch (const InvalidArgument &) {
      // a caller mistake, found before any device work
      err_slot_put(j->err);
      throw;
    } catch (...) {
      // work already queued may still write the slot: let it land first,
      // and leave the lane's word clear for the next job
      discard_err(p, p->execs[lane]);
      err_slot_put(j->err);
      if (j->done) (void)hipEventDestroy(j->done);
      throw;
    }
    p->next = (p->next + 1) % (int)p->execs.size();
    *job = j.release();
  });
}

int cchip_job_wait(cchip_job *j) {
  if (j->waited) {
    if (j->status) set_last_error(j->msg);
    return j->status;
  }
  int rc = guarded([&] {
    cchip_program *p = j->prog;
    DeviceGuard dg(p->device);
    check_hip(hipEventSynchronize(j->done), "hipEventSynchronize");
    std::lock_guard<std::mutex> lk(p->mu);
    if (p->released) return;
    raise_err_slot(p, j->err);
  });
  j->waited = true;
  j->status = rc;
  if (rc) j->msg = cchip_last_error();
  return rc;
}

int cchip_job_free(cchip_job *j) {
  if (!j) return 0;
  if (j->done) {
    // the slot is written by the job's own stream: recycle it only once
    // that copy has landed
    (void)hipEventSynchronize(j->done);
    (void)hipEventDestroy(j->done);
  }
  err_slot_put(j->err);
  delete j;
  return 0;
}

int cchip_program_run_resident(cchip_program *p, int n, const char *const *names, void *const *dev_inputs,
                               const size_t *bytes, void **outputs) {
  return guarded([&] {
    std::lock_guard<std::mutex> lk(p->mu);
    DeviceGuard dg(p->device);
    run_resident_impl(p, n, names, dev_inputs, bytes, outputs, nullptr, true);
  });
}

int cchip_program_run_resident_into(cchip_program *p, int n, const char *const *names, void *const *dev_inputs,
                                    const size_t *bytes, void *const *dev_outputs, int sync) {
  return guarded([&] {
    std::lock_guard<std::mutex> lk(p->mu);
    DeviceGuard dg(p->device);
    run_resident_impl(p, n, names, dev_inputs, bytes, nullptr, dev_outputs, sync != 0);
  });
}

int cchip_program_run_resident_noalloc(cchip_program *p, int n, const char *const *names, void *const *dev_inputs,
                                       const size_t *bytes, void *const *dev_outputs, void *stream, int *err_out) {
  return guarded([&] {
    std::lock_guard<std::mutex> lk(p->mu);
    if (p->released) throw Failure("Executor.run_resident: this executor has been released");
    const ProgramIR &ir = p->ir;
    const size_t cap = noalloc_scratch_capacity();
    if (p->na_bytes > (int64_t)cap)
      throw InvalidArgument(strf("run_resident_noalloc: program %s needs %lld bytes of scratch, more than the "
                                 "%zu bytes of the static scratch",
                                 ir.name.c_str(), (long long)p->na_bytes, cap));
    // inputs by name, exact byte sizes, before any device work
    for (size_t k = 0; k < ir.params.size(); k++) {
      const IOSpec &ps = ir.params[k];
      int w = -1;
      for (int i = 0; i < n && w < 0; i++)
        if (names[i] && ps.name == names[i]) w = i;
      if (w < 0) throw InvalidArgument("Executor.run_resident: missing input " + ps.name);
      if (bytes[w] != (size_t)ir.bufs[ps.buf].bytes())
        throw InvalidArgument(strf("Executor.run_resident: input %s is %zu bytes, parameter %s needs %lld",
                                   ps.name.c_str(), bytes[w], ir.bufs[ps.buf].name.c_str(),
                                   (long long)ir.bufs[ps.buf].bytes()));
      p->na_which[k] = w;
    }
    DeviceGuard dg(p->device);
    char *base = (char *)noalloc_scratch(p->device);
    const Executor &e = p->execs[0];
    for (size_t b = 0; b < ir.bufs.size(); b++)
      p->na_ptr[b] = p->na_off[b] >= 0 ? (void *)(base + p->na_off[b]) : e.bufs[b];
    for (size_t k = 0; k < ir.params.size(); k++) p->na_ptr[ir.params[k].buf] = dev_inputs[p->na_which[k]];
    for (size_t o = 0; o < ir.outputs.size(); o++)
      if (!p->na_out_copy[o]) p->na_ptr[ir.outputs[o].buf] = dev_outputs[o];
    hipStream_t st = (hipStream_t)stream;
    // the scratch starts at zero, as a fresh pool does
    noalloc_scratch_clear(base, (size_t)p->na_bytes, stream);
    for (auto &op : ir.plan) {
      if (op.kind != OpK::Launch) continue;
      const KernelSpec &k = ir.kernels[op.kernel];
      for (size_t i = 0; i < k.args.size(); i++) {
        p->na_vals[i] = p->na_ptr[k.args[i]];
        p->na_args[i] = &p->na_vals[i];
      }
      check_hip(hipModuleLaunchKernel((hipFunction_t)p->kfn[op.kernel], k.grid, k.grid_y, 1, k.block, k.block_y, 1,
                                      k.shared_bytes, st, p->na_args.data(), nullptr),
                "hipModuleLaunchKernel");
    }
    for (size_t o = 0; o < ir.outputs.size(); o++) {
      if (!p->na_out_copy[o]) continue;
      size_t nb = (size_t)ir.bufs[ir.outputs[o].buf].bytes();
      if (nb)
        check_hip(hipMemcpyAsync(dev_outputs[o], p->na_ptr[ir.outputs[o].buf], nb, hipMemcpyDeviceToDevice, st),
                  "copy_device");
    }
    // this call's error word (the first word of the static scratch, cleared
    // above with the rest), for the caller to read after synchronising
    if (err_out)
      check_hip(hipMemcpyAsync(err_out, base, sizeof(int), hipMemcpyDeviceToDevice, st), "copy error word");
  });
}

int cchip_error_word_status(int code) {
  return guarded([&] {
    if (code) throw InvalidArgument(err_message(code));
  });
}

int cchip_program_stream(const cchip_program *p, int lane, void **stream) {
  return guarded([&] {
    if (lane < 0 || lane >= (int)p->execs.size()) throw InvalidArgument("no such lane");
    *stream = p->execs[lane].stream;
  });
}

int cchip_program_time_kernel(cchip_program *p, const char *name) {
  return guarded([&] {
    std::lock_guard<std::mutex> lk(p->mu);
    p->timed = -1;
    if (!name) return;
    for (size_t k = 0; k < p->ir.kernels.size(); k++)
      if (p->ir.kernels[k].name == name) p->timed = (int)k;
    if (p->timed < 0) throw InvalidArgument(std::string("no kernel named ") + name);
    for (auto &e : p->ev_used) p->ev_free.push_back(e);
    p->ev_used.clear();
  });
}

int cchip_program_timing_each(cchip_program *p, int capacity, double *each_ms, int *launches, double *total_ms) {
  return guarded([&] {
    std::lock_guard<std::mutex> lk(p->mu);
    DeviceGuard dg(p->device);
    double tot = 0;
    int i = 0;
    for (auto &e : p->ev_used) {
      check_hip(hipEventSynchronize(e.second), "hipEventSynchronize");
      float ms = 0;
      check_hip(hipEventElapsedTime(&ms, e.first, e.second), "hipEventElapsedTime");
      tot += ms;
      if (each_ms && i < capacity) each_ms[i] = ms;
      i++;
    }
    *launches = (int)p->ev_used.size();
    *total_ms = tot;
    for (auto &e : p->ev_used) p->ev_free.push_back(e);
    p->ev_used.clear();
  });
}

int cchip_program_timing(cchip_program *p, int *launches, double *total_ms) {
  return cchip_program_timing_each(p, 0, nullptr, launches, total_ms);
}

}  // extern "C"
