// lib/runtime over HIP: device, buffers with a live count, streams, events,
// hiprtc JIT with a code-object cache, launch and pinned host memory.
// Restates the behaviour of lib/runtime/*.ml (device.ml:32-122,
// buffer.ml:11-79, stream.ml:8-25, event.ml:7-15, jit.ml:11-36,
// launch.ml:9-13, pinned.ml:13-118) on the HIP module API.

#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <mutex>
#include <set>
#include <sstream>
#include <sys/stat.h>
#include <unistd.h>

#include "../../include/cchip_runtime.h"
#include "internal.hpp"

namespace cchip {

static thread_local std::string g_last_error;

void set_last_error(const std::string &msg) { g_last_error = msg; }

std::string strf(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  char buf[2048];
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return buf;
}

const char *dt_name(DT d) {
  switch (d) {
    case DT::F32: return "f32";
    case DT::F64: return "f64";
    case DT::I32: return "i32";
    case DT::I64: return "i64";
    default: return "bool";
  }
}

const char *dt_ctype(DT d) {
  switch (d) {
    case DT::F32: return "float";
    case DT::F64: return "double";
    case DT::I32: return "int";
    case DT::I64: return "long long";
    default: return "bool";
  }
}

void check_hip(int status, const char *what) {
  if (status != hipSuccess)
    throw Failure(strf("hip: %s: %s", what, hipGetErrorString(static_cast<hipError_t>(status))));
}

static std::once_flag g_init_once;
static int g_init_status = hipSuccess;

void ensure_init() {
  std::call_once(g_init_once, [] { g_init_status = hipInit(0); });
  check_hip(g_init_status, "hipInit");
}

static std::atomic<int64_t> g_live{0};

void *rt_alloc(size_t bytes) {
  ensure_init();
  void *p = nullptr;
  check_hip(hipMalloc(&p, bytes == 0 ? 1 : bytes), "hipMalloc");
  g_live++;
  return p;
}

void rt_free(void *p) {
  if (!p) return;
  check_hip(hipFree(p), "hipFree");
  g_live--;
}

// ---------------------------------------------------------------------------
// JIT: hiprtc -> code object -> hipModuleLoadData, with an in-process and an
// on-disk cache keyed by a hash of (options, source).
// ---------------------------------------------------------------------------

static const char *const kJitOptions[] = {
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    // Every interpreter operation is rounded separately; no a*b+c contraction.
    "-ffp-contract=off",
    // Keep the compiler from forming packed-FP32 instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-rdc",
};

static uint64_t fnv1a(const std::string &s, uint64_t h = 1469598103934665603ull) {
  for (unsigned char c : s) {
    h ^= c;
    h *= 1099511628211ull;
  }
  return h;
}

// The on-disk cache directory, or "" when it must not be used: it has to be
// a real directory owned by this user and writable by nobody else, so code
// objects are only ever loaded from a directory this process controls.
static std::string cache_dir() {
  const char *env = getenv("CCHIP_CACHE_DIR");
  std::string d = env && *env ? env : "/tmp/cchip-jit-cache";
  mkdir(d.c_str(), 0700);
  struct stat st;
  if (lstat(d.c_str(), &st) != 0 || !S_ISDIR(st.st_mode) || st.st_uid != geteuid() ||
      (st.st_mode & (S_IWGRP | S_IWOTH)))
    return "";
  return d;
}

// What the code objects depend on beyond the source and the options: the
// hiprtc (compiler) version, so a toolchain update never loads stale code.
static std::string compiler_tag() {
  int major = 0, minor = 0;
  if (hiprtcVersion(&major, &minor) != HIPRTC_SUCCESS) major = minor = -1;
  return strf("hiprtc %d.%d gfx950", major, minor);
}

static std::mutex g_jit_mu;
static std::map<uint64_t, std::vector<char>> g_co_cache;

std::vector<char> jit_code_object(const std::string &name, const std::string &source) {
  std::string opts = compiler_tag() + " ";
  for (const char *o : kJitOptions) opts += std::string(o) + " ";
  uint64_t key = fnv1a(source, fnv1a(opts));
  {
    std::lock_guard<std::mutex> lk(g_jit_mu);
    auto it = g_co_cache.find(key);
    if (it != g_co_cache.end()) return it->second;
  }
  const char *nocache = getenv("CCHIP_NO_DISK_CACHE");
  const std::string dir = nocache && *nocache == '1' ? std::string() : cache_dir();
  const bool disk = !dir.empty();
  std::string path = dir + strf("/%016llx.co", (unsigned long long)key);
  if (disk) {
    std::ifstream in(path, std::ios::binary);
    if (in) {
      std::vector<char> co((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
      if (!co.empty()) {
        std::lock_guard<std::mutex> lk(g_jit_mu);
        g_co_cache[key] = co;
        return co;
      }
    }
  }
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, source.c_str(), (name + ".hip").c_str(), 0, nullptr, nullptr) != HIPRTC_SUCCESS)
    throw Failure("hiprtc: cannot create program " + name);
  int nopt = sizeof(kJitOptions) / sizeof(kJitOptions[0]);
  hiprtcResult rc = hiprtcCompileProgram(prog, nopt, kJitOptions);
  size_t logsz = 0;
  hiprtcGetProgramLogSize(prog, &logsz);
  std::string log(logsz, '\0');
  if (logsz) hiprtcGetProgramLog(prog, &log[0]);
  if (rc != HIPRTC_SUCCESS) {
    hiprtcDestroyProgram(&prog);
    throw Failure("hiprtc: " + name + ": " + hiprtcGetErrorString(rc) + "\n" + log);
  }
  size_t cs = 0;
  hiprtcGetCodeSize(prog, &cs);
  std::vector<char> co(cs);
  hiprtcGetCode(prog, co.data());
  hiprtcDestroyProgram(&prog);
  if (disk) {
    std::string tmp = path + strf(".%d.tmp", (int)getpid());
    std::ofstream out(tmp, std::ios::binary);
    if (out) {
      out.write(co.data(), (std::streamsize)co.size());
      out.close();
      rename(tmp.c_str(), path.c_str());
    }
  }
  std::lock_guard<std::mutex> lk(g_jit_mu);
  g_co_cache[key] = co;
  return co;
}

struct Module {
  hipModule_t mod = nullptr;
  size_t code_bytes = 0;
  std::map<std::string, hipFunction_t> fns;
  ~Module() {
    if (mod) (void)hipModuleUnload(mod);
  }
};

std::shared_ptr<Module> jit_compile(const std::string &name, const std::string &source) {
  ensure_init();
  std::vector<char> co = jit_code_object(name, source);
  auto m = std::make_shared<Module>();
  check_hip(hipModuleLoadData(&m->mod, co.data()), "hipModuleLoadData");
  m->code_bytes = co.size();
  return m;
}

void *module_kernel(Module &m, const std::string &name) {
  auto it = m.fns.find(name);
  if (it != m.fns.end()) return (void *)it->second;
  hipFunction_t f = nullptr;
  if (hipModuleGetFunction(&f, m.mod, name.c_str()) != hipSuccess || !f)
    throw Failure("jit: no kernel named " + name);
  m.fns[name] = f;
  return (void *)f;
}

}  // namespace cchip

using namespace cchip;

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------

extern "C" {

const char *cchip_last_error(void) { return g_last_error.c_str(); }

int cchip_device_available(void) {
  int n = 0;
  if (hipInit(0) != hipSuccess) return 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n > 0 ? 1 : 0;
}

int cchip_device_init(void) {
  return guarded([] {
    ensure_init();
    int n = 0;
    check_hip(hipGetDeviceCount(&n), "hipGetDeviceCount");
    if (n < 1) throw Failure("hip: no device");
    int cur = 0;
    check_hip(hipGetDevice(&cur), "hipGetDevice");
    check_hip(hipSetDevice(cur), "hipSetDevice");
  });
}

int cchip_device_synchronize(void) {
  return guarded([] { check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize"); });
}

int cchip_device_count(int *count) {
  return guarded([&] {
    ensure_init();
    int n = 0;
    check_hip(hipGetDeviceCount(&n), "hipGetDeviceCount");
    *count = n;
  });
}

int cchip_device_get(int *ordinal) {
  return guarded([&] {
    ensure_init();
    check_hip(hipGetDevice(ordinal), "hipGetDevice");
  });
}

int cchip_device_set(int ordinal) {
  return guarded([&] {
    ensure_init();
    int n = 0;
    check_hip(hipGetDeviceCount(&n), "hipGetDeviceCount");
    if (ordinal < 0 || ordinal >= n) throw InvalidArgument(strf("Device.with_device: no device %d", ordinal));
    check_hip(hipSetDevice(ordinal), "hipSetDevice");
  });
}

int cchip_device_info(int ordinal, char *name, size_t name_len, char *arch, size_t arch_len, int *mps,
                      int64_t *mem) {
  return guarded([&] {
    ensure_init();
    int n = 0;
    check_hip(hipGetDeviceCount(&n), "hipGetDeviceCount");
    if (ordinal < 0 || ordinal >= n) throw InvalidArgument(strf("Device.info_of: no device %d", ordinal));
    hipDeviceProp_t p;
    check_hip(hipGetDeviceProperties(&p, ordinal), "hipGetDeviceProperties");
    // "gfx950:sramecc+:xnack-" -> "gfx950"
    std::string a = p.gcnArchName;
    size_t c = a.find(':');
    if (c != std::string::npos) a = a.substr(0, c);
    if (name && name_len) {
      // Some drivers report no marketing name; Device.name is never empty
      // (device.mli), so fall back to hipDeviceGetName, then to the
      // architecture.
      std::string nm = p.name;
      if (nm.empty()) {
        char buf[256] = {0};
        if (hipDeviceGetName(buf, sizeof buf - 1, ordinal) == hipSuccess) nm = buf;
      }
      if (nm.empty()) nm = "AMD " + a;
      snprintf(name, name_len, "%s", nm.c_str());
    }
    if (arch && arch_len) snprintf(arch, arch_len, "%s", a.c_str());
    if (mps) *mps = p.multiProcessorCount;
    if (mem) *mem = (int64_t)p.totalGlobalMem;
  });
}

int cchip_buffer_alloc(size_t bytes, void **dptr) {
  return guarded([&] { *dptr = rt_alloc(bytes); });
}

int cchip_buffer_free(void *dptr) {
  return guarded([&] { rt_free(dptr); });
}

int64_t cchip_buffer_live_count(void) { return g_live.load(); }

int cchip_buffer_upload(void *dst, const void *src, size_t bytes) {
  return guarded([&] {
    if (bytes) check_hip(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
  });
}

int cchip_buffer_download(void *dst, const void *src, size_t bytes) {
  return guarded([&] {
    if (bytes) check_hip(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
  });
}

int cchip_buffer_upload_async(void *dst, const void *src, size_t bytes, void *stream) {
  return guarded([&] {
    if (bytes)
      check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream), "hipMemcpyAsync H2D");
  });
}

int cchip_buffer_download_async(void *dst, const void *src, size_t bytes, void *stream) {
  return guarded([&] {
    if (bytes)
      check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream), "hipMemcpyAsync D2H");
  });
}

int cchip_buffer_copy_device(void *dst, const void *src, size_t bytes, void *stream) {
  return guarded([&] {
    if (bytes)
      check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream), "hipMemcpyAsync D2D");
  });
}

int cchip_stream_create(void **stream) {
  return guarded([&] {
    ensure_init();
    hipStream_t s;
    check_hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags");
    *stream = s;
  });
}

int cchip_stream_destroy(void *stream) {
  return guarded([&] {
    if (stream) check_hip(hipStreamDestroy((hipStream_t)stream), "hipStreamDestroy");
  });
}

int cchip_stream_synchronize(void *stream) {
  return guarded([&] { check_hip(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize"); });
}

int cchip_stream_is_idle(void *stream, int *idle) {
  return guarded([&] {
    hipError_t e = hipStreamQuery((hipStream_t)stream);
    if (e == hipSuccess) *idle = 1;
    else if (e == hipErrorNotReady) *idle = 0;
    else check_hip(e, "hipStreamQuery");
  });
}

int cchip_event_record(void *stream, void **event) {
  return guarded([&] {
    ensure_init();
    hipEvent_t e;
    check_hip(hipEventCreate(&e), "hipEventCreate");
    check_hip(hipEventRecord(e, (hipStream_t)stream), "hipEventRecord");
    *event = e;
  });
}

int cchip_event_wait(void *stream, void *event) {
  return guarded([&] { check_hip(hipStreamWaitEvent((hipStream_t)stream, (hipEvent_t)event, 0), "hipStreamWaitEvent"); });
}

int cchip_event_synchronize(void *event) {
  return guarded([&] { check_hip(hipEventSynchronize((hipEvent_t)event), "hipEventSynchronize"); });
}

int cchip_event_elapsed_ms(void *start, void *stop, float *ms) {
  return guarded(
      [&] { check_hip(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop), "hipEventElapsedTime"); });
}

int cchip_event_destroy(void *event) {
  return guarded([&] { check_hip(hipEventDestroy((hipEvent_t)event), "hipEventDestroy"); });
}

// Modules handed across the C ABI are owned by this table.
static std::mutex g_mod_mu;
static std::map<void *, std::shared_ptr<Module>> g_modules;

int cchip_jit_compile(const char *name, const char *source, void **module) {
  return guarded([&] {
    auto m = jit_compile(name, source);
    std::lock_guard<std::mutex> lk(g_mod_mu);
    g_modules[m.get()] = m;
    *module = m.get();
  });
}

int cchip_jit_check(const char *name, const char *source, size_t *code_bytes) {
  return guarded([&] {
    std::vector<char> co = jit_code_object(name, source);
    if (code_bytes) *code_bytes = co.size();
  });
}

int cchip_jit_code_size(void *module, size_t *bytes) {
  return guarded([&] {
    if (!module) throw InvalidArgument("Jit: null module");
    *bytes = ((Module *)module)->code_bytes;
  });
}

int cchip_jit_get_kernel(void *module, const char *name, void **kernel) {
  return guarded([&] {
    if (!module) throw InvalidArgument("Jit: null module");
    *kernel = module_kernel(*(Module *)module, name);
  });
}

int cchip_jit_unload(void *module) {
  return guarded([&] {
    std::lock_guard<std::mutex> lk(g_mod_mu);
    g_modules.erase(module);
  });
}

int cchip_launch(void *kernel, int grid, int grid_y, int block, int block_y, int shared_bytes, void *stream, int nargs,
                 void *const *dev_ptrs) {
  return guarded([&] {
    if (grid < 1 || grid_y < 1 || block < 1 || block_y < 1 || block * block_y > 1024)
      throw InvalidArgument(strf("Launch.run: bad geometry %dx%d / %dx%d", grid, grid_y, block, block_y));
    std::vector<void *> vals(dev_ptrs, dev_ptrs + nargs);
    std::vector<void *> args(nargs);
    for (int i = 0; i < nargs; i++) args[i] = &vals[i];
    check_hip(hipModuleLaunchKernel((hipFunction_t)kernel, grid, grid_y, 1, block, block_y, 1, shared_bytes,
                                    (hipStream_t)stream, args.data(), nullptr),
              "hipModuleLaunchKernel");
  });
}

static std::mutex g_pin_mu;
static std::set<const void *> g_pinned;

int cchip_pinned_alloc(size_t bytes, void **host) {
  return guarded([&] {
    ensure_init();
    void *p = nullptr;
    check_hip(hipHostMalloc(&p, bytes ? bytes : 1, hipHostMallocPortable), "hipHostMalloc");
    memset(p, 0, bytes ? bytes : 1);
    std::lock_guard<std::mutex> lk(g_pin_mu);
    g_pinned.insert(p);
    *host = p;
  });
}

int cchip_pinned_free(void *host) {
  return guarded([&] {
    {
      std::lock_guard<std::mutex> lk(g_pin_mu);
      if (!g_pinned.erase(host)) throw InvalidArgument("Pinned: not a pinned allocation");
    }
    check_hip(hipHostFree(host), "hipHostFree");
  });
}

int cchip_pinned_is_pinned(const void *host) {
  std::lock_guard<std::mutex> lk(g_pin_mu);
  return g_pinned.count(host) ? 1 : 0;
}

}  // extern "C"
