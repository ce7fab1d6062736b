// libnewt_hip.so - the C-ABI backend boundary of newt on MI355X (gfx950).
//
// Replaces the reference's ctypes bindings to NVRTC and the CUDA driver API
// (newt/runtime/cuda.py): hipRTC compiles generated HIP C++ to a code object,
// the HIP module API loads it and launches it on the caller's stream.
//
// hipRTC is not linked: it is opened at first use from the directory of the
// libamdhip64 this process already runs with (torch-ROCm ships a matching
// hipRTC + comgr pair next to its HIP runtime), so the compiler that produces
// code objects always belongs to the runtime that loads them.
#include <hip/hip_runtime.h>
#include <dlfcn.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/newt_hip.h"

namespace {

thread_local std::string g_last_error;

int fail(int status, const std::string& msg) {
  g_last_error = msg;
  return status;
}

int hip_fail(hipError_t e, const char* what) {
  std::string msg = std::string(what) + ": " + hipGetErrorName(e) + " (" +
                    hipGetErrorString(e) + ")";
  return fail(static_cast<int>(e), msg);
}

// ---- hipRTC, resolved at run time ------------------------------------------
typedef int rtc_status;
typedef void* rtc_program;
struct RtcApi {
  rtc_status (*create)(rtc_program*, const char*, const char*, int, const char**,
                       const char**);
  rtc_status (*compile)(rtc_program, int, const char**);
  rtc_status (*log_size)(rtc_program, size_t*);
  rtc_status (*log)(rtc_program, char*);
  rtc_status (*code_size)(rtc_program, size_t*);
  rtc_status (*code)(rtc_program, char*);
  rtc_status (*destroy)(rtc_program*);
  const char* (*error_string)(rtc_status);
  rtc_status (*version)(int*, int*);
  void* handle = nullptr;
  std::string path;
};

std::once_flag g_rtc_once;
RtcApi g_rtc;
std::string g_rtc_error;

std::string dir_of_hip_runtime() {
  Dl_info info;
  if (dladdr(reinterpret_cast<void*>(&hipModuleLoadData), &info) && info.dli_fname) {
    std::string p(info.dli_fname);
    size_t slash = p.rfind('/');
    if (slash != std::string::npos) return p.substr(0, slash);
  }
  return std::string();
}

void load_rtc() {
  std::vector<std::string> candidates;
  const char* env = std::getenv("NEWT_HIPRTC_LIBRARY");
  if (env && *env) candidates.push_back(env);
  std::string dir = dir_of_hip_runtime();
  if (!dir.empty()) {
    candidates.push_back(dir + "/libhiprtc.so");
    candidates.push_back(dir + "/libhiprtc.so.7");
  }
  candidates.push_back("libhiprtc.so.7");
  candidates.push_back("libhiprtc.so");
  std::string errors;
  for (const auto& c : candidates) {
    void* h = dlopen(c.c_str(), RTLD_NOW | RTLD_LOCAL);
    if (!h) {
      const char* e = dlerror();
      errors += c + ": " + (e ? e : "?") + "\n";
      continue;
    }
    RtcApi api;
    api.handle = h;
    api.path = c;
    bool ok = true;
#define NEWT_SYM(field, name)                                               \
  *reinterpret_cast<void**>(&api.field) = dlsym(h, name);                   \
  if (!api.field) { ok = false; errors += c + ": missing " name "\n"; }
    NEWT_SYM(create, "hiprtcCreateProgram")
    NEWT_SYM(compile, "hiprtcCompileProgram")
    NEWT_SYM(log_size, "hiprtcGetProgramLogSize")
    NEWT_SYM(log, "hiprtcGetProgramLog")
    NEWT_SYM(code_size, "hiprtcGetCodeSize")
    NEWT_SYM(code, "hiprtcGetCode")
    NEWT_SYM(destroy, "hiprtcDestroyProgram")
    NEWT_SYM(error_string, "hiprtcGetErrorString")
    NEWT_SYM(version, "hiprtcVersion")
#undef NEWT_SYM
    if (ok) {
      g_rtc = api;
      return;
    }
    dlclose(h);
  }
  g_rtc_error = "newt: could not load hipRTC\n" + errors;
}

const RtcApi* rtc() {
  std::call_once(g_rtc_once, load_rtc);
  return g_rtc.handle ? &g_rtc : nullptr;
}

}  // namespace

struct newt_module_s {
  hipModule_t mod;
};
struct newt_function_s {
  hipFunction_t fn;
};

extern "C" {

int newt_abi_version(void) { return NEWT_ABI_VERSION; }

const char* newt_error_string(int status) {
  switch (status) {
    case NEWT_OK: return "success";
    case NEWT_ERR_RTC: return "hipRTC compilation failed";
    case NEWT_ERR_INVALID: return "invalid argument";
    case NEWT_ERR_NOT_FOUND: return "kernel symbol not found";
    default: break;
  }
  if (status > 0 && status < 10000) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown newt status";
}

const char* newt_last_error(void) { return g_last_error.c_str(); }

void newt_free(void* p) { std::free(p); }

int newt_rtc_version(int* version) {
  const RtcApi* api = rtc();
  if (!api) return fail(NEWT_ERR_RTC, g_rtc_error);
  if (!version) return fail(NEWT_ERR_INVALID, "newt_rtc_version: null output");
  int major = 0, minor = 0;
  rtc_status s = api->version(&major, &minor);
  if (s != 0) return fail(NEWT_ERR_RTC, api->error_string(s));
  *version = major * 100 + minor;
  return NEWT_OK;
}

int newt_rtc_compile(const char* source, const char* name, const char* arch,
                     const char* const* options, int num_options,
                     const char* const* headers, const char* const* header_names,
                     int num_headers, void** code, size_t* code_size) {
  if (!source || !name || !code || !code_size || num_options < 0 || num_headers < 0)
    return fail(NEWT_ERR_INVALID, "newt_rtc_compile: null argument");
  *code = nullptr;
  *code_size = 0;
  const RtcApi* api = rtc();
  if (!api) return fail(NEWT_ERR_RTC, g_rtc_error);
  rtc_program prog = nullptr;
  rtc_status s = api->create(&prog, source, name, num_headers,
                             const_cast<const char**>(headers),
                             const_cast<const char**>(header_names));
  if (s != 0) return fail(NEWT_ERR_RTC, std::string("hiprtcCreateProgram: ") + api->error_string(s));
  std::vector<std::string> opts;
  if (arch && *arch) opts.push_back(std::string("--offload-arch=") + arch);
  for (int i = 0; i < num_options; ++i)
    if (options[i]) opts.emplace_back(options[i]);
  std::vector<const char*> copts;
  for (auto& o : opts) copts.push_back(o.c_str());
  s = api->compile(prog, static_cast<int>(copts.size()), copts.data());
  size_t log_size = 0;
  std::string log;
  if (api->log_size(prog, &log_size) == 0 && log_size > 1) {
    log.resize(log_size);
    api->log(prog, &log[0]);
    log.resize(std::strlen(log.c_str()));
  }
  if (s != 0) {
    std::string msg = std::string("hipRTC error: ") + api->error_string(s) + "\n" + log;
    api->destroy(&prog);
    return fail(NEWT_ERR_RTC, msg);
  }
  size_t n = 0;
  s = api->code_size(prog, &n);
  if (s != 0 || n == 0) {
    api->destroy(&prog);
    return fail(NEWT_ERR_RTC, "hipRTC produced no code object\n" + log);
  }
  void* buf = std::malloc(n);
  if (!buf) {
    api->destroy(&prog);
    return fail(NEWT_ERR_INVALID, "out of host memory");
  }
  s = api->code(prog, static_cast<char*>(buf));
  api->destroy(&prog);
  if (s != 0) {
    std::free(buf);
    return fail(NEWT_ERR_RTC, std::string("hiprtcGetCode: ") + api->error_string(s));
  }
  *code = buf;
  *code_size = n;
  g_last_error = log;  // warnings, if any
  return NEWT_OK;
}

int newt_module_load(const void* image, size_t size, newt_module_t* module) {
  if (!image || size == 0 || !module) return fail(NEWT_ERR_INVALID, "newt_module_load: bad image");
  hipModule_t m = nullptr;
  hipError_t e = hipModuleLoadData(&m, image);
  if (e != hipSuccess) return hip_fail(e, "hipModuleLoadData");
  *module = new newt_module_s{m};
  return NEWT_OK;
}

int newt_module_get_function(newt_module_t module, const char* name,
                             newt_function_t* function) {
  if (!module || !name || !function) return fail(NEWT_ERR_INVALID, "newt_module_get_function: null argument");
  hipFunction_t f = nullptr;
  hipError_t e = hipModuleGetFunction(&f, module->mod, name);
  if (e == hipErrorNotFound) return fail(NEWT_ERR_NOT_FOUND, std::string("no kernel named ") + name);
  if (e != hipSuccess) return hip_fail(e, "hipModuleGetFunction");
  *function = new newt_function_s{f};
  return NEWT_OK;
}

int newt_module_unload(newt_module_t module) {
  if (!module) return fail(NEWT_ERR_INVALID, "newt_module_unload: null module");
  hipError_t e = hipModuleUnload(module->mod);
  delete module;
  if (e != hipSuccess) return hip_fail(e, "hipModuleUnload");
  return NEWT_OK;
}

int newt_function_set_max_lds(newt_function_t function, int bytes) {
  if (!function || bytes < 0) return fail(NEWT_ERR_INVALID, "newt_function_set_max_lds: bad argument");
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  int limit = 0;
  e = hipDeviceGetAttribute(&limit, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
  if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute");
  if (bytes > limit)
    return fail(NEWT_ERR_INVALID, "kernel needs " + std::to_string(bytes) +
                                      " bytes of LDS, device allows " + std::to_string(limit));
  // HIP imposes no opt-in threshold for dynamic LDS below the device limit.
  return NEWT_OK;
}

int newt_function_attributes(newt_function_t function, int* num_regs, int* lds_bytes,
                             int* scratch_bytes, int* max_threads) {
  if (!function) return fail(NEWT_ERR_INVALID, "newt_function_attributes: null function");
  struct Q { int* out; hipFunction_attribute a; } qs[] = {
      {num_regs, HIP_FUNC_ATTRIBUTE_NUM_REGS},
      {lds_bytes, HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES},
      {scratch_bytes, HIP_FUNC_ATTRIBUTE_LOCAL_SIZE_BYTES},
      {max_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK}};
  for (auto& q : qs) {
    if (!q.out) continue;
    hipError_t e = hipFuncGetAttribute(q.out, q.a, function->fn);
    if (e != hipSuccess) return hip_fail(e, "hipFuncGetAttribute");
  }
  return NEWT_OK;
}

int newt_launch(newt_function_t function, unsigned gx, unsigned gy, unsigned gz,
                unsigned block, unsigned lds_bytes, void* stream, void** args) {
  if (!function) return fail(NEWT_ERR_INVALID, "newt_launch: null function");
  if (block == 0 || block > 1024 || gx == 0 || gy == 0 || gz == 0)
    return fail(NEWT_ERR_INVALID, "newt_launch: bad launch shape");
  hipError_t e = hipModuleLaunchKernel(function->fn, gx, gy, gz, block, 1, 1, lds_bytes,
                                       static_cast<hipStream_t>(stream), args, nullptr);
  if (e != hipSuccess) return hip_fail(e, "hipModuleLaunchKernel");
  return NEWT_OK;
}

int newt_launch_packed(newt_function_t function, unsigned gx, unsigned gy, unsigned gz,
                       unsigned block, unsigned lds_bytes, void* stream,
                       const void* argbuf, size_t argsize) {
  if (!function) return fail(NEWT_ERR_INVALID, "newt_launch_packed: null function");
  if (block == 0 || block > 1024 || gx == 0 || gy == 0 || gz == 0)
    return fail(NEWT_ERR_INVALID, "newt_launch_packed: bad launch shape");
  size_t size = argsize;
  // A kernel without parameters still needs a valid (empty) buffer pointer.
  static const unsigned long long empty = 0;
  void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER,
                    const_cast<void*>(argsize ? argbuf : &empty),
                    HIP_LAUNCH_PARAM_BUFFER_SIZE, &size, HIP_LAUNCH_PARAM_END};
  hipError_t e = hipModuleLaunchKernel(function->fn, gx, gy, gz, block, 1, 1, lds_bytes,
                                       static_cast<hipStream_t>(stream), nullptr, config);
  if (e != hipSuccess) return hip_fail(e, "hipModuleLaunchKernel");
  return NEWT_OK;
}

// libamdhip64's launch with events recorded by the dispatch packet (declared
// here: hip_ext.h also holds templates that need the HIP compiler, and this
// file is plain C++)
extern "C" hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t globalWorkSizeX,
                                               uint32_t globalWorkSizeY, uint32_t globalWorkSizeZ,
                                               uint32_t localWorkSizeX, uint32_t localWorkSizeY,
                                               uint32_t localWorkSizeZ, size_t sharedMemBytes,
                                               hipStream_t hStream, void** kernelParams,
                                               void** extra, hipEvent_t startEvent,
                                               hipEvent_t stopEvent, uint32_t flags);

int newt_launch_packed_timed(newt_function_t function, unsigned gx, unsigned gy, unsigned gz,
                             unsigned block, unsigned lds_bytes, void* stream,
                             const void* argbuf, size_t argsize, void* ev_start,
                             void* ev_stop) {
  if (!function) return fail(NEWT_ERR_INVALID, "newt_launch_packed_timed: null function");
  if (block == 0 || block > 1024 || gx == 0 || gy == 0 || gz == 0)
    return fail(NEWT_ERR_INVALID, "newt_launch_packed_timed: bad launch shape");
  // this launch API takes work-item counts, not workgroup counts
  if ((unsigned long long)gx * block > 0xffffffffull)
    return fail(NEWT_ERR_INVALID, "newt_launch_packed_timed: grid too large");
  size_t size = argsize;
  static const unsigned long long empty = 0;
  void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER,
                    const_cast<void*>(argsize ? argbuf : &empty),
                    HIP_LAUNCH_PARAM_BUFFER_SIZE, &size, HIP_LAUNCH_PARAM_END};
  hipError_t e = hipExtModuleLaunchKernel(function->fn, gx * block, gy, gz, block, 1, 1,
                                          lds_bytes, static_cast<hipStream_t>(stream),
                                          nullptr, config, static_cast<hipEvent_t>(ev_start),
                                          static_cast<hipEvent_t>(ev_stop), 0);
  if (e != hipSuccess) return hip_fail(e, "hipExtModuleLaunchKernel");
  return NEWT_OK;
}

int newt_device_arch(int device, char* buf, size_t buflen) {
  if (!buf || buflen == 0) return fail(NEWT_ERR_INVALID, "newt_device_arch: null buffer");
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
  std::snprintf(buf, buflen, "%s", prop.gcnArchName);
  return NEWT_OK;
}

int newt_device_limits(int device, int* num_cus, int* max_lds_per_block, int* warp_size) {
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
  if (num_cus) *num_cus = prop.multiProcessorCount;
  if (max_lds_per_block) *max_lds_per_block = static_cast<int>(prop.sharedMemPerBlock);
  if (warp_size) *warp_size = prop.warpSize;
  return NEWT_OK;
}

}  // extern "C"
