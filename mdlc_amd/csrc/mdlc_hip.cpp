// libmdlc_hip.so — hipRTC + HIP module runtime for the fused-group backend.
// The C ABI is declared (with the reference interface each entry replaces)
// in include/mdlc_hip.h.
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <hip/hiprtc.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "mdlc_hip.h"

// The allocation-free plan runner's workspace (mdlc_plan_run_static): a
// file-scope device array, one copy per GPU, held until the process ends.
// Host code never uses its name as an address: mdlc_init resolves each
// device's copy with hipGetSymbolAddress and keeps the pointer per device.
constexpr size_t kStaticScratchBytes = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {

std::string g_err;
hipStream_t g_stream = nullptr;
int g_device = -1;
constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};

enum ShimCode : int { kBadArg = 9001, kBadPlan = 9002 };

int fail(int code, const char* what, const char* detail) {
  char buf[512];
  std::snprintf(buf, sizeof(buf), "%s failed with code %d: %s", what, code,
                detail ? detail : "");
  g_err = buf;
  return code == 0 ? kBadArg : code;
}

int check(hipError_t e, const char* what) {
  if (e == hipSuccess) return 0;
  return fail(static_cast<int>(e), what, hipGetErrorString(e));
}

int need_stream(const char* what) {
  if (g_stream == nullptr) return fail(kBadArg, what, "mdlc_init has not been called");
  return 0;
}

struct Launch {
  hipFunction_t fn;
  unsigned grid[3];
  unsigned block[3];
  unsigned lds;
  std::vector<uint64_t> blob;    // argument values, 8-byte slots
  std::vector<void*> argv;       // pointers into blob, one per argument
  // workspace arguments (plan format 2): blob slot and offset into the
  // workspace; the static runner's copy of the values, rebased on the
  // device's static scratch at each call
  std::vector<size_t> ws_slot;
  std::vector<uint64_t> ws_off;
  std::vector<uint64_t> sblob;
  std::vector<void*> sargv;
};

struct Plan {
  std::vector<Launch> launches;
  bool use_graph = false;
  hipGraphExec_t exec = nullptr;
  hipGraph_t graph = nullptr;
  uint64_t ws_base = 0;          // the caller's workspace (0: none bound)
  uint64_t ws_bytes = 0;         // workspace the plan's kernels use
  bool has_ws = false;           // some argument is a workspace pointer
};

// A plan whose workspace arguments have no caller workspace behind them can
// only run on the static scratch.
int need_workspace(const Plan* p, const char* what) {
  if (p->has_ws && p->ws_base == 0)
    return fail(kBadPlan, what, "the plan has no workspace bound; run it with mdlc_plan_run_static");
  return 0;
}

int enqueue(Launch& l) {
  return check(hipModuleLaunchKernel(l.fn, l.grid[0], l.grid[1], l.grid[2], l.block[0],
                                     l.block[1], l.block[2], l.lds, g_stream,
                                     l.argv.data(), nullptr),
               "hipModuleLaunchKernel");
}

int enqueue_plan(Plan* p) {
  int rc = need_workspace(p, "mdlc_plan_run");
  if (rc) return rc;
  if (p->use_graph && p->exec != nullptr)
    return check(hipGraphLaunch(p->exec, g_stream), "hipGraphLaunch");
  for (auto& l : p->launches) {
    rc = enqueue(l);
    if (rc) return rc;
  }
  return 0;
}

void drop_graph(Plan* p) {
  if (p->exec) hipGraphExecDestroy(p->exec);
  if (p->graph) hipGraphDestroy(p->graph);
  p->exec = nullptr;
  p->graph = nullptr;
}

template <typename T>
bool take(const uint8_t*& cur, const uint8_t* end, T* out) {
  if (static_cast<size_t>(end - cur) < sizeof(T)) return false;
  std::memcpy(out, cur, sizeof(T));
  cur += sizeof(T);
  return true;
}

}  // namespace

extern "C" {

const char* mdlc_last_error(void) { return g_err.c_str(); }

int mdlc_device_count(int* count) {
  if (!count) return fail(kBadArg, "mdlc_device_count", "null count");
  *count = 0;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) return check(e, "hipGetDeviceCount");
  *count = n;
  return 0;
}

int mdlc_init(int device, char* arch, int arch_len) {
  int rc = check(hipSetDevice(device), "hipSetDevice");
  if (rc) return rc;
  if (g_stream == nullptr || g_device != device) {
    if (g_stream != nullptr) hipStreamDestroy(g_stream);
    rc = check(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking), "hipStreamCreate");
    if (rc) return rc;
    g_device = device;
  }
  if (device >= 0 && device < kMaxDevices && g_scratch_ptr[device] == nullptr) {
    void* ptr = nullptr;
    rc = check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (rc) return rc;
    g_scratch_ptr[device] = ptr;
  }
  if (arch && arch_len > 0) {
    hipDeviceProp_t prop;
    rc = check(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    if (rc) return rc;
    std::string name(prop.gcnArchName);
    name = name.substr(0, name.find(':'));
    std::snprintf(arch, static_cast<size_t>(arch_len), "%s", name.c_str());
  }
  return 0;
}

int mdlc_rtc_compile(const char* src, const char* name, const char* const* opts, int nopts,
                     void** code, size_t* size, char* log, size_t log_len) {
  if (!src || !code || !size) return fail(kBadArg, "mdlc_rtc_compile", "null argument");
  *code = nullptr;
  *size = 0;
  if (log && log_len) log[0] = '\0';
  hiprtcProgram prog;
  hiprtcResult r = hiprtcCreateProgram(&prog, src, name ? name : "kernels.hip", 0, nullptr, nullptr);
  if (r != HIPRTC_SUCCESS) return fail(static_cast<int>(r), "hiprtcCreateProgram", hiprtcGetErrorString(r));
  r = hiprtcCompileProgram(prog, nopts, const_cast<const char**>(opts));
  size_t ln = 0;
  if (hiprtcGetProgramLogSize(prog, &ln) == HIPRTC_SUCCESS && ln > 1 && log && log_len) {
    std::vector<char> buf(ln + 1, '\0');
    hiprtcGetProgramLog(prog, buf.data());
    std::snprintf(log, log_len, "%s", buf.data());
  }
  if (r != HIPRTC_SUCCESS) {
    int rc = fail(static_cast<int>(r), "hiprtcCompileProgram", hiprtcGetErrorString(r));
    hiprtcDestroyProgram(&prog);
    return rc;
  }
  size_t n = 0;
  r = hiprtcGetCodeSize(prog, &n);
  if (r != HIPRTC_SUCCESS || n == 0) {
    hiprtcDestroyProgram(&prog);
    return fail(r == HIPRTC_SUCCESS ? kBadArg : static_cast<int>(r), "hiprtcGetCodeSize", "empty code object");
  }
  void* buf = std::malloc(n);
  if (!buf) {
    hiprtcDestroyProgram(&prog);
    return fail(kBadArg, "mdlc_rtc_compile", "host allocation failed");
  }
  r = hiprtcGetCode(prog, static_cast<char*>(buf));
  hiprtcDestroyProgram(&prog);
  if (r != HIPRTC_SUCCESS) {
    std::free(buf);
    return fail(static_cast<int>(r), "hiprtcGetCode", hiprtcGetErrorString(r));
  }
  *code = buf;
  *size = n;
  return 0;
}

void mdlc_rtc_free(void* code) { std::free(code); }

int mdlc_rtc_version(int* rtc_major, int* rtc_minor, int* runtime) {
  if (!rtc_major || !rtc_minor || !runtime) return fail(kBadArg, "mdlc_rtc_version", "null argument");
  hiprtcResult r = hiprtcVersion(rtc_major, rtc_minor);
  if (r != HIPRTC_SUCCESS) return fail(static_cast<int>(r), "hiprtcVersion", hiprtcGetErrorString(r));
  return check(hipRuntimeGetVersion(runtime), "hipRuntimeGetVersion");
}

int mdlc_module_load(const void* code, size_t size, void** module) {
  (void)size;
  if (!code || !module) return fail(kBadArg, "mdlc_module_load", "null argument");
  hipModule_t m = nullptr;
  int rc = check(hipModuleLoadData(&m, code), "hipModuleLoadData");
  if (rc) return rc;
  *module = m;
  return 0;
}

int mdlc_get_function(void* module, const char* name, void** function) {
  if (!module || !name || !function) return fail(kBadArg, "mdlc_get_function", "null argument");
  hipFunction_t f = nullptr;
  hipError_t e = hipModuleGetFunction(&f, static_cast<hipModule_t>(module), name);
  if (e != hipSuccess) return fail(static_cast<int>(e), "hipModuleGetFunction", name);
  *function = f;
  return 0;
}

int mdlc_module_unload(void* module) {
  return check(hipModuleUnload(static_cast<hipModule_t>(module)), "hipModuleUnload");
}

int mdlc_malloc(size_t nbytes, void** ptr) {
  if (!ptr) return fail(kBadArg, "mdlc_malloc", "null ptr");
  return check(hipMalloc(ptr, nbytes ? nbytes : 1), "hipMalloc");
}

int mdlc_free(void* ptr) { return check(hipFree(ptr), "hipFree"); }

static int copy(void* dst, const void* src, size_t n, hipMemcpyKind kind, const char* what) {
  int rc = need_stream(what);
  if (rc) return rc;
  if (n == 0) return 0;
  rc = check(hipMemcpyAsync(dst, src, n, kind, g_stream), what);
  if (rc) return rc;
  return check(hipStreamSynchronize(g_stream), what);
}

int mdlc_memcpy_htod(void* dst, const void* src, size_t n) {
  return copy(dst, src, n, hipMemcpyHostToDevice, "mdlc_memcpy_htod");
}
int mdlc_memcpy_dtoh(void* dst, const void* src, size_t n) {
  return copy(dst, src, n, hipMemcpyDeviceToHost, "mdlc_memcpy_dtoh");
}
int mdlc_memcpy_dtod(void* dst, const void* src, size_t n) {
  return copy(dst, src, n, hipMemcpyDeviceToDevice, "mdlc_memcpy_dtod");
}

int mdlc_launch(void* function, unsigned gx, unsigned gy, unsigned gz, unsigned bx, unsigned by,
                unsigned bz, unsigned lds_bytes, void** args) {
  int rc = need_stream("mdlc_launch");
  if (rc) return rc;
  return check(hipModuleLaunchKernel(static_cast<hipFunction_t>(function), gx, gy, gz, bx, by, bz,
                                     lds_bytes, g_stream, args, nullptr),
               "hipModuleLaunchKernel");
}

int mdlc_sync(void) {
  int rc = need_stream("mdlc_sync");
  if (rc) return rc;
  return check(hipStreamSynchronize(g_stream), "hipStreamSynchronize");
}

int mdlc_event_create(void** event) {
  hipEvent_t e = nullptr;
  int rc = check(hipEventCreate(&e), "hipEventCreate");
  if (!rc) *event = e;
  return rc;
}
int mdlc_event_destroy(void* event) {
  return check(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy");
}
int mdlc_event_record(void* event) {
  int rc = need_stream("mdlc_event_record");
  if (rc) return rc;
  return check(hipEventRecord(static_cast<hipEvent_t>(event), g_stream), "hipEventRecord");
}
int mdlc_event_elapsed_ms(void* start, void* stop, float* ms) {
  int rc = check(hipEventSynchronize(static_cast<hipEvent_t>(stop)), "hipEventSynchronize");
  if (rc) return rc;
  return check(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)),
               "hipEventElapsedTime");
}

int mdlc_plan_create(const void* packed, size_t nbytes, void** plan) {
  if (!packed || !plan) return fail(kBadArg, "mdlc_plan_create", "null argument");
  const uint8_t* cur = static_cast<const uint8_t*>(packed);
  const uint8_t* end = cur + nbytes;
  char magic[4];
  uint32_t version = 0, n = 0, reserved = 0;
  if (!take(cur, end, &magic) || std::memcmp(magic, "MDLP", 4) != 0 || !take(cur, end, &version) ||
      (version != 1 && version != 2) || !take(cur, end, &n) || !take(cur, end, &reserved))
    return fail(kBadPlan, "mdlc_plan_create", "bad header");
  Plan* p = new Plan();
  if (version == 2 && (!take(cur, end, &p->ws_base) || !take(cur, end, &p->ws_bytes))) {
    delete p;
    return fail(kBadPlan, "mdlc_plan_create", "bad header");
  }
  p->launches.resize(n);
  for (uint32_t i = 0; i < n; ++i) {
    Launch& l = p->launches[i];
    uint64_t fn = 0;
    uint32_t nargs = 0;
    bool ok = take(cur, end, &fn);
    for (int d = 0; d < 3 && ok; ++d) ok = take(cur, end, &l.grid[d]);
    for (int d = 0; d < 3 && ok; ++d) ok = take(cur, end, &l.block[d]);
    ok = ok && take(cur, end, &l.lds) && take(cur, end, &nargs);
    if (!ok || fn == 0) {
      delete p;
      return fail(kBadPlan, "mdlc_plan_create", "truncated launch record");
    }
    l.fn = reinterpret_cast<hipFunction_t>(fn);
    std::vector<size_t> slot(nargs);
    for (uint32_t a = 0; a < nargs; ++a) {
      uint32_t sz = 0;
      if (!take(cur, end, &sz)) {
        delete p;
        return fail(kBadPlan, "mdlc_plan_create", "bad argument size");
      }
      // format 2: the top bit marks a workspace pointer given as an offset
      const bool ws = version == 2 && (sz & 0x80000000u);
      sz &= 0x7fffffffu;
      if (sz == 0 || sz > 64 || (ws && sz != 8)) {
        delete p;
        return fail(kBadPlan, "mdlc_plan_create", "bad argument size");
      }
      size_t padded = (sz + 7) / 8 * 8;
      if (static_cast<size_t>(end - cur) < padded) {
        delete p;
        return fail(kBadPlan, "mdlc_plan_create", "truncated argument");
      }
      slot[a] = l.blob.size();
      l.blob.resize(l.blob.size() + padded / 8, 0);
      std::memcpy(l.blob.data() + slot[a], cur, sz);
      cur += padded;
      if (ws) {
        const uint64_t off = l.blob[slot[a]];
        if (off >= p->ws_bytes) {
          delete p;
          return fail(kBadPlan, "mdlc_plan_create", "workspace offset outside the workspace");
        }
        l.ws_slot.push_back(slot[a]);
        l.ws_off.push_back(off);
        l.blob[slot[a]] = p->ws_base ? p->ws_base + off : 0;
        p->has_ws = true;
      }
    }
    l.argv.resize(nargs);
    for (uint32_t a = 0; a < nargs; ++a) l.argv[a] = l.blob.data() + slot[a];
    l.sblob = l.blob;
    l.sargv.resize(nargs);
    for (uint32_t a = 0; a < nargs; ++a) l.sargv[a] = l.sblob.data() + slot[a];
  }
  *plan = p;
  return 0;
}

int mdlc_plan_destroy(void* plan) {
  Plan* p = static_cast<Plan*>(plan);
  if (p) {
    drop_graph(p);
    delete p;
  }
  return 0;
}

int mdlc_plan_num_launches(void* plan, int* n) {
  if (!plan || !n) return fail(kBadArg, "mdlc_plan_num_launches", "null argument");
  *n = static_cast<int>(static_cast<Plan*>(plan)->launches.size());
  return 0;
}

int mdlc_plan_run(void* plan, int iters) {
  int rc = need_stream("mdlc_plan_run");
  if (rc) return rc;
  Plan* p = static_cast<Plan*>(plan);
  for (int i = 0; i < iters; ++i) {
    rc = enqueue_plan(p);
    if (rc) return rc;
  }
  return 0;
}

int mdlc_plan_run_static(void* plan, int iters) {
  int rc = need_stream("mdlc_plan_run_static");
  if (rc) return rc;
  Plan* p = static_cast<Plan*>(plan);
  if (!p || iters < 0) return fail(kBadArg, "mdlc_plan_run_static", "bad arguments");
  if (p->ws_bytes > kStaticScratchBytes) {
    char buf[160];
    std::snprintf(buf, sizeof(buf), "the plan's workspace of %llu bytes exceeds the static scratch of %llu bytes",
                  static_cast<unsigned long long>(p->ws_bytes),
                  static_cast<unsigned long long>(kStaticScratchBytes));
    return fail(kBadArg, "mdlc_plan_run_static", buf);
  }
  void* base = (g_device >= 0 && g_device < kMaxDevices) ? g_scratch_ptr[g_device] : nullptr;
  if (base == nullptr) return fail(kBadArg, "mdlc_plan_run_static", "no static scratch on this device");
  for (int it = 0; it < iters; ++it) {
    for (auto& l : p->launches) {
      for (size_t j = 0; j < l.ws_slot.size(); ++j)
        l.sblob[l.ws_slot[j]] = reinterpret_cast<uint64_t>(base) + l.ws_off[j];
      rc = check(hipModuleLaunchKernel(l.fn, l.grid[0], l.grid[1], l.grid[2], l.block[0], l.block[1],
                                       l.block[2], l.lds, g_stream, l.sargv.data(), nullptr),
                 "hipModuleLaunchKernel");
      if (rc) return rc;
    }
  }
  return 0;
}

int mdlc_plan_time_ms(void* plan, int warmup, int iters, float* ms) {
  if (!ms || iters <= 0) return fail(kBadArg, "mdlc_plan_time_ms", "bad arguments");
  int rc = mdlc_plan_run(plan, warmup);
  if (rc) return rc;
  hipEvent_t a = nullptr, b = nullptr;
  if ((rc = check(hipEventCreate(&a), "hipEventCreate"))) return rc;
  if ((rc = check(hipEventCreate(&b), "hipEventCreate"))) {
    hipEventDestroy(a);
    return rc;
  }
  rc = check(hipEventRecord(a, g_stream), "hipEventRecord");
  if (!rc) rc = mdlc_plan_run(plan, iters);
  if (!rc) rc = check(hipEventRecord(b, g_stream), "hipEventRecord");
  if (!rc) rc = check(hipEventSynchronize(b), "hipEventSynchronize");
  float t = 0.f;
  if (!rc) rc = check(hipEventElapsedTime(&t, a, b), "hipEventElapsedTime");
  hipEventDestroy(a);
  hipEventDestroy(b);
  if (!rc) *ms = t / static_cast<float>(iters);
  return rc;
}

int mdlc_plan_profile(void* plan, int iters, float* per_launch_ms) {
  int rc = need_stream("mdlc_plan_profile");
  if (rc) return rc;
  Plan* p = static_cast<Plan*>(plan);
  if (!per_launch_ms || iters <= 0) return fail(kBadArg, "mdlc_plan_profile", "bad arguments");
  if ((rc = need_workspace(p, "mdlc_plan_profile"))) return rc;
  size_t n = p->launches.size();
  // the events ride on each kernel's own dispatch (hipExtModuleLaunchKernel),
  // so they time the kernel's execution, not the queue's work around it;
  // the `iters` runs of the plan are enqueued back to back (one wait at the
  // end: a wait per run would start each run's first kernel on an idle
  // device), and a launch's figure is the median of its `iters` times
  const size_t runs = static_cast<size_t>(iters);
  std::vector<hipEvent_t> ev(2 * n * runs, nullptr);
  for (auto& e : ev)
    if ((rc = check(hipEventCreate(&e), "hipEventCreate"))) break;
  std::vector<float> samples(n * runs, 0.f);
  for (size_t it = 0; it < runs && !rc; ++it) {
    for (size_t i = 0; i < n && !rc; ++i) {
      Launch& l = p->launches[i];
      hipEvent_t* e = &ev[2 * (it * n + i)];
      rc = check(hipExtModuleLaunchKernel(l.fn, l.grid[0] * l.block[0], l.grid[1] * l.block[1],
                                          l.grid[2] * l.block[2], l.block[0], l.block[1],
                                          l.block[2], l.lds, g_stream, l.argv.data(), nullptr,
                                          e[0], e[1], 0),
                 "hipExtModuleLaunchKernel");
    }
  }
  if (!rc) rc = check(hipStreamSynchronize(g_stream), "hipStreamSynchronize");
  for (size_t it = 0; it < runs && !rc; ++it)
    for (size_t i = 0; i < n && !rc; ++i)
      rc = check(hipEventElapsedTime(&samples[i * runs + it], ev[2 * (it * n + i)],
                                     ev[2 * (it * n + i) + 1]),
                 "hipEventElapsedTime");
  for (size_t i = 0; i < n && !rc; ++i) {
    float* s = &samples[i * iters];
    std::sort(s, s + iters);
    per_launch_ms[i] = iters % 2 ? s[iters / 2] : 0.5f * (s[iters / 2 - 1] + s[iters / 2]);
  }
  for (auto& e : ev)
    if (e) hipEventDestroy(e);
  return rc;
}

int mdlc_plan_use_graph(void* plan, int enable) {
  int rc = need_stream("mdlc_plan_use_graph");
  if (rc) return rc;
  Plan* p = static_cast<Plan*>(plan);
  if (!enable) {
    p->use_graph = false;
    return 0;
  }
  if ((rc = need_workspace(p, "mdlc_plan_use_graph"))) return rc;
  if (p->exec == nullptr) {
    rc = check(hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    if (rc) return rc;
    for (auto& l : p->launches) {
      rc = enqueue(l);
      if (rc) break;
    }
    hipGraph_t g = nullptr;
    int rc2 = check(hipStreamEndCapture(g_stream, &g), "hipStreamEndCapture");
    if (rc || rc2) {
      if (g) hipGraphDestroy(g);
      return rc ? rc : rc2;
    }
    p->graph = g;
    rc = check(hipGraphInstantiate(&p->exec, g, nullptr, nullptr, 0), "hipGraphInstantiate");
    if (rc) {
      drop_graph(p);
      return rc;
    }
  }
  p->use_graph = true;
  return 0;
}

}  // extern "C"
