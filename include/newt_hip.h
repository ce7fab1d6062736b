/*
 * newt_hip.h - C ABI of libnewt_hip.so, the MI355X (gfx950) backend boundary of newt.
 *
 * The reference backend is a ctypes binding to two NVIDIA libraries
 * (newt/runtime/cuda.py): NVRTC for source -> cubin and the CUDA driver API for
 * module load and launch. This header is the drop-in replacement for exactly that
 * boundary: hipRTC for source -> gfx950 code object, the HIP module API for load
 * and launch. Everything crosses as plain pointers, sizes and C strings; no torch
 * or HIP types appear in the signatures (streams and device pointers are void*).
 *
 * Error convention: every function returns 0 on success or a nonzero status.
 * Codes below 10000 are hipError_t values; NEWT_ERR_* are this library's own.
 * newt_error_string() turns any of them into text; newt_last_error() returns the
 * detailed message of the last failure on the calling thread (e.g. the hipRTC
 * build log), mirroring NVRTCError / CUDAError (newt/runtime/cuda.py:101-121,
 * :161-174).
 */
#ifndef NEWT_HIP_H
#define NEWT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NEWT_ABI_VERSION 1

#define NEWT_OK 0
#define NEWT_ERR_RTC 10001        /* hipRTC compile failed; log in newt_last_error() */
#define NEWT_ERR_INVALID 10002    /* bad argument (null handle, bad size, ...) */
#define NEWT_ERR_NOT_FOUND 10003  /* kernel symbol not present in the code object */

typedef struct newt_module_s* newt_module_t;
typedef struct newt_function_s* newt_function_t;

/* Library ABI version (NEWT_ABI_VERSION). No reference counterpart. */
int newt_abi_version(void);

/* Text for a status code returned by any newt_* call.
 * Replaces: _cu_check / cuGetErrorString (newt/runtime/cuda.py:165-174). */
const char* newt_error_string(int status);

/* Detailed message of the last failure on this thread ("" if none). */
const char* newt_last_error(void);

/* Compile HIP C++ source to a gfx950 code object with hipRTC.
 * `headers`/`header_names` supply in-memory includes (num_headers entries).
 * On success *code / *code_size hold a malloc'd image (free with newt_free).
 * On NEWT_ERR_RTC the build log is returned by newt_last_error().
 * Replaces: compile_cuda (newt/runtime/cuda.py:124-154). */
int newt_rtc_compile(const char* source, const char* name, const char* arch,
                     const char* const* options, int num_options,
                     const char* const* headers, const char* const* header_names,
                     int num_headers, void** code, size_t* code_size);

/* hipRTC version as major*100+minor (part of the code-object cache key).
 * Replaces: the NVRTC version implied by _load_nvrtc (newt/runtime/cuda.py:44-62). */
int newt_rtc_version(int* version);

/* Release memory returned by this library. */
void newt_free(void* p);

/* Load a code object into the current device's context.
 * Replaces: cuModuleLoadData in Kernel.__init__ (newt/runtime/cuda.py:198-201). */
int newt_module_load(const void* image, size_t size, newt_module_t* module);

/* Look up an extern "C" __global__ function by name.
 * Replaces: cuModuleGetFunction (newt/runtime/cuda.py:202-205). */
int newt_module_get_function(newt_module_t module, const char* name,
                             newt_function_t* function);

/* Unload a module (the JIT keeps modules for the process lifetime, as the
 * reference does; provided for completeness and tests). */
int newt_module_unload(newt_module_t module);

/* Allow up to `bytes` of dynamic LDS for the function.
 * Replaces: cuFuncSetAttribute(MAX_DYNAMIC_SHARED_SIZE_BYTES) (cuda.py:206-213). */
int newt_function_set_max_lds(newt_function_t function, int bytes);

/* Static resource usage of a loaded function (registers, LDS, scratch), for
 * the structural tests and the autotuner. No reference counterpart. */
int newt_function_attributes(newt_function_t function, int* num_regs,
                             int* lds_bytes, int* scratch_bytes, int* max_threads);

/* Launch with an array of pointers to argument values (CUDA driver style).
 * grid is (gx, gy, gz) workgroups, `block` threads (64 * waves), `lds_bytes`
 * of dynamic LDS, on `stream` (a hipStream_t, NULL = default stream).
 * Replaces: Kernel.launch -> cuLaunchKernel (newt/runtime/cuda.py:216-234). */
int newt_launch(newt_function_t function, unsigned gx, unsigned gy, unsigned gz,
                unsigned block, unsigned lds_bytes, void* stream, void** args);

/* Launch with the kernel arguments already packed into one buffer laid out as
 * the kernel's argument segment (natural alignment of each parameter). One call
 * from Python instead of one ctypes object per argument: the per-launch host
 * path of the JIT (newt/runtime/jit.py:190-223) uses this. */
int newt_launch_packed(newt_function_t function, unsigned gx, unsigned gy,
                       unsigned gz, unsigned block, unsigned lds_bytes,
                       void* stream, const void* argbuf, size_t argsize);

/* newt_launch_packed, with two HIP events (hipEvent_t, either may be NULL)
 * that the dispatch itself records when the kernel starts and ends
 * (hipExtModuleLaunchKernel): per-launch kernel times without separate
 * event-record packets between back-to-back launches. No reference
 * counterpart; bench.py times its launches with it. */
int newt_launch_packed_timed(newt_function_t function, unsigned gx, unsigned gy,
                             unsigned gz, unsigned block, unsigned lds_bytes,
                             void* stream, const void* argbuf, size_t argsize,
                             void* ev_start, void* ev_stop);

/* gcnArchName of a device (e.g. "gfx950:sramecc+:xnack-") into buf.
 * Replaces: _arch() / torch.cuda.get_device_capability (newt/runtime/jit.py:26-32). */
int newt_device_arch(int device, char* buf, size_t buflen);

/* Number of compute units and LDS bytes per workgroup of a device (autotune
 * space sizing). No reference counterpart. */
int newt_device_limits(int device, int* num_cus, int* max_lds_per_block,
                       int* warp_size);

#ifdef __cplusplus
}
#endif

#endif /* NEWT_HIP_H */
