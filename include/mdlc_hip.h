/*
 * mdlc_hip.h — C ABI of libmdlc_hip.so, the MI355X device runtime behind the
 * fused-group codegen path.
 *
 * It replaces the reference's ctypes bindings to NVRTC and the CUDA driver in
 * mdlc/codegen/cuda/nvrtc_runtime.py. Each entry point below names the
 * reference function it stands in for. Plain pointers and sizes only; every
 * function returns 0 on success or a nonzero hipError_t / hiprtcResult /
 * shim code, and mdlc_last_error() then describes the failure.
 *
 * Threading: one host thread drives the library. All launches, copies and
 * events go to the single stream created by mdlc_init (the reference used
 * the default stream, nvrtc_runtime.py:157, :218-221). Not thread-safe.
 */
#ifndef MDLC_HIP_H
#define MDLC_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Message for the most recent failure ("" if none).
 * Replaces: CudaError text built by _ck/_ckn, nvrtc_runtime.py:74-92. */
const char* mdlc_last_error(void);

/* Number of visible HIP devices (0 and a nonzero code when none).
 * Replaces: the device-count probe in cuda_available(), nvrtc_runtime.py:57-71. */
int mdlc_device_count(int* count);

/* Select `device`, create the library's stream, and write the device's ISA
 * name (e.g. "gfx950") into arch[0..arch_len).
 * Replaces: CudaContext.__init__ / _compute_arch, nvrtc_runtime.py:165-180. */
int mdlc_init(int device, char* arch, int arch_len);

/* hipRTC-compile `src` to a code object. On success *code is a malloc'd
 * buffer of *size bytes (release with mdlc_rtc_free). The build log (also on
 * failure) is copied into log[0..log_len).
 * Replaces: compile_to_ptx, nvrtc_runtime.py:97-124. */
int mdlc_rtc_compile(const char* src, const char* name, const char* const* opts, int nopts,
                     void** code, size_t* size, char* log, size_t log_len);
void mdlc_rtc_free(void* code);

/* hipRTC's version and the HIP runtime's (hipRuntimeGetVersion), neither of
 * which needs a device. No counterpart in the reference (it caches nothing):
 * the Python side keys its on-disk code-object cache on them, so objects built
 * by another toolchain are never reused. */
int mdlc_rtc_version(int* rtc_major, int* rtc_minor, int* runtime);

/* Load a code object / resolve a kernel / unload.
 * Replaces: cuModuleLoadData and CudaModule.func, nvrtc_runtime.py:133-144. */
int mdlc_module_load(const void* code, size_t size, void** module);
int mdlc_get_function(void* module, const char* name, void** function);
int mdlc_module_unload(void* module);

/* Device memory. Copies are ordered on the library stream and complete
 * before return.
 * Replaces: CudaContext.malloc/free/to_device/from_device, nvrtc_runtime.py:183-202. */
int mdlc_malloc(size_t nbytes, void** ptr);
int mdlc_free(void* ptr);
int mdlc_memcpy_htod(void* dst, const void* src, size_t nbytes);
int mdlc_memcpy_dtoh(void* dst, const void* src, size_t nbytes);
int mdlc_memcpy_dtod(void* dst, const void* src, size_t nbytes);

/* Enqueue one kernel on the library stream. args[i] points at the i-th
 * kernel argument's value (the hipModuleLaunchKernel convention).
 * Replaces: CudaModule.launch / cuLaunchKernel, nvrtc_runtime.py:146-159. */
int mdlc_launch(void* function, unsigned gx, unsigned gy, unsigned gz,
                unsigned bx, unsigned by, unsigned bz, unsigned lds_bytes, void** args);

/* Wait for the library stream.
 * Replaces: CudaContext.synchronize / cuCtxSynchronize, nvrtc_runtime.py:204-205. */
int mdlc_sync(void);

/* Events on the library stream, for timing.
 * Replaces: the cuEvent* calls inside CudaContext.time_ms, nvrtc_runtime.py:211-225. */
int mdlc_event_create(void** event);
int mdlc_event_destroy(void* event);
int mdlc_event_record(void* event);
int mdlc_event_elapsed_ms(void* start, void* stop, float* ms);

/* Packed launch plans: the executor's launch loop in C++.
 * Replaces: the Python `issue()` loop of GpuExecutor.run, gpu_executor.py:63-91.
 *
 * Layout (little endian): "MDLP", u32 version (1 or 2), u32 n_launches,
 * u32 0; version 2 adds u64 ws_base, u64 ws_bytes (the workspace the plan's
 * kernels use: split-K partial sums, stream-K pieces, column matrices);
 * then per launch: u64 function, u32 grid[3], u32 block[3], u32 lds_bytes,
 * u32 n_args, then per argument u32 nbytes followed by the value bytes,
 * zero-padded to a multiple of 8. In version 2 an nbytes with its top bit
 * set (0x80000000 | 8) marks a workspace pointer whose value is an offset
 * below ws_bytes; the plan passes ws_base + offset. A version-2 plan with
 * ws_base 0 has no workspace of its own and runs only through
 * mdlc_plan_run_static (the other entries refuse it).
 *
 * mdlc_plan_run enqueues every launch `iters` times without waiting.
 * mdlc_plan_time_ms brackets `iters` runs (after `warmup` runs) with events.
 * mdlc_plan_profile times each launch's kernel execution with a start and
 * stop event attached to its own dispatch (hipExtModuleLaunchKernel), over
 * `iters` runs of the plan, and writes each launch's median into
 * per_launch_ms[0..n_launches).
 * mdlc_plan_use_graph(plan, 1) captures the plan once into a hipGraph and
 * replays that graph from then on (0 returns to direct launches). */
int mdlc_plan_create(const void* packed, size_t nbytes, void** plan);
int mdlc_plan_destroy(void* plan);
int mdlc_plan_num_launches(void* plan, int* n);
int mdlc_plan_run(void* plan, int iters);
int mdlc_plan_time_ms(void* plan, int warmup, int iters, float* ms);
int mdlc_plan_profile(void* plan, int iters, float* per_launch_ms);
int mdlc_plan_use_graph(void* plan, int enable);

/* mdlc_plan_run without a caller workspace: the plan's workspace pointers
 * are rebased on the library's static scratch, a file-scope device array of
 * 64 MiB per GPU that mdlc_init resolves once per device and that is held
 * until the process ends. Allocates nothing (no hipMalloc, hipFree or
 * allocating library call), so callers that cannot allocate device memory
 * (code being captured into a HIP graph, tight serving loops, harnesses that
 * forbid it) can run a plan. A plan whose ws_bytes exceeds 64 MiB is refused
 * with an error. Every call on one GPU shares that GPU's array and leaves
 * its contents behind; the kernels write every workspace element they read
 * in the same call, so nothing needs clearing. Calls that overlap on one GPU
 * (another thread or process running a plan on it at the same time) race.
 * No counterpart in the reference: its executor allocated every buffer per
 * run (gpu_executor.py:48-61); this entry is for the callers that cannot
 * allocate. */
int mdlc_plan_run_static(void* plan, int iters);

#ifdef __cplusplus
}
#endif

#endif /* MDLC_HIP_H */
