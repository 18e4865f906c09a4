/* vesta_hip.h -- C ABI of the Vesta HIP runtime shim (libvesta_hip.so).
 *
 * The shim is the native boundary of the decode hot path: run-time
 * compilation of a generated kernel with hipRTC for gfx950, module loading,
 * occupancy and device queries, and one cooperative launch per decode step.
 * Python reaches it through ctypes (vesta/launch.py). Plain pointers and
 * sizes only; device buffers are owned by the caller (torch), the shim owns
 * only module handles and the buffers it returns from vh_compile.
 *
 * Every call returns a status: 0 on success, otherwise a code that
 * vh_error_string() names. Codes 1..9999 are hipError_t values, codes
 * 10000 + k are hiprtcResult k, codes >= 20000 are the shim's own.
 *
 * Reference interface each entry point replaces (reference tree vesta/):
 *   vh_compile                    launch.py:17-27   compile_cubin (NVRTC)
 *   vh_module_load                launch.py:34      cuModuleLoadData
 *   vh_module_get_function        launch.py:35      cuModuleGetFunction
 *   vh_function_set_dynamic_lds   launch.py:36-39   cuFuncSetAttribute(MAX_DYNAMIC_SHARED)
 *   vh_occupancy                  launch.py:40-41   cuOccupancyMaxActiveBlocksPerMultiprocessor
 *   vh_device_info                launch.py:32,43   device capability / multiprocessor count
 *   vh_launch_cooperative         launch.py:68-70   cuLaunchCooperativeKernel
 *   vh_module_unload, vh_function_attrs, vh_free, vh_error_string,
 *   vh_synchronize, vh_launch: no counterpart (the reference never unloads or queries).
 */
#ifndef VESTA_HIP_H
#define VESTA_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VH_OK 0
#define VH_ERR_RTC_BASE 10000
#define VH_ERR_NULL_ARG 20001
#define VH_ERR_NO_COOP 20002
#define VH_ERR_BAD_OCCUPANCY 20003
#define VH_ERR_SCRATCH_TOO_SMALL 20004

/* Compile `src` (HIP C++) with hipRTC. `opts` are compiler options such as
 * "--offload-arch=gfx950" and "-O3". On success *code / *code_size hold the
 * code object (free with vh_free). *log receives the compile log (possibly
 * empty, free with vh_free) whether or not compilation succeeded; pass NULL
 * to skip it. */
int vh_compile(const char* src, const char* name, const char* const* opts, int nopts,
               void** code, size_t* code_size, char** log);

/* Release a buffer returned by vh_compile. */
void vh_free(void* p);

/* Load a code object on the current device; *module is an opaque handle. */
int vh_module_load(const void* code, void** module);

/* Look up a kernel by its (extern "C") name; *fn is an opaque handle. */
int vh_module_get_function(void* module, const char* name, void** fn);

/* Unload a module; its functions become invalid. */
int vh_module_unload(void* module);

/* Allow `bytes` of dynamic LDS per workgroup for `fn`. */
int vh_function_set_dynamic_lds(void* fn, int bytes);

/* Registers (VGPRs per lane as the runtime reports them), static LDS bytes,
 * private (spill/scratch) bytes per lane and the largest block size of `fn`. */
int vh_function_attrs(void* fn, int* regs, int* static_lds, int* private_bytes, int* max_block);

/* Workgroups of `block` threads with `dyn_lds` bytes of dynamic LDS that can
 * be resident on one CU at once. */
int vh_occupancy(void* fn, int block, size_t dyn_lds, int* per_cu);

/* Compute units, cooperative-launch support (0/1), LDS bytes per workgroup
 * and the architecture name (e.g. "gfx950:sramecc+:xnack-") of device `dev`. */
int vh_device_info(int dev, int* cu_count, int* coop, int* lds_per_block, char* arch, size_t arch_len);

/* One cooperative launch of `fn` on `stream` (a hipStream_t, may be NULL for
 * the null stream). `args` is the kernel argument array: args[i] points at the
 * value of argument i; it is read before the call returns. */
int vh_launch_cooperative(void* fn, unsigned grid, unsigned block, unsigned dyn_lds, void* stream, void** args);

/* One ordinary (non-cooperative) launch, same arguments. For kernels that
 * do not wait on other blocks, and (profiling only, where a profiler's
 * teardown fails after cooperative launches) for a persistent kernel whose
 * grid is at most one block per CU on an otherwise idle device: its grid
 * barriers' bounded waits end a launch whose blocks are not all resident.
 * No counterpart in the reference. */
int vh_launch(void* fn, unsigned grid, unsigned block, unsigned dyn_lds, void* stream, void** args);

/* ---- Allocation-free launch. No counterpart in the reference: for callers
 * that cannot allocate device memory (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc). The kernel's scratch `S`, barrier
 * counters `bar` and timing sums `TS` (three consecutive kernel arguments)
 * live in one static device array of VH_NOALLOC_SCRATCH_BYTES per device,
 * held until the process ends; the caller still passes every residue. */
#define VH_NOALLOC_SCRATCH_BYTES (8u << 20)
#define VH_NOALLOC_MAX_ARGS 64

/* Device address and size of the current device's static scratch. */
int vh_noalloc_scratch(void** base, size_t* bytes);

/* Where bar and TS start in the static scratch for buffers of these sizes (S
 * at 0, each start 256-byte aligned); VH_ERR_SCRATCH_TOO_SMALL beyond it. */
int vh_noalloc_layout(size_t s_bytes, size_t bar_bytes, size_t ts_bytes, size_t* bar_off, size_t* ts_off);

/* Copy `bytes` of the static scratch from `offset` to device memory `dst`,
 * ordered on `stream` (outputs a launch left in S, such as the logits). */
int vh_noalloc_read(void* dst, size_t offset, size_t bytes, void* stream);

/* vh_launch_cooperative with args[slot], args[slot + 1], args[slot + 2]
 * replaced by the static scratch's S, bar and TS (s_bytes, bar_bytes,
 * ts_bytes long; VH_ERR_SCRATCH_TOO_SMALL when they do not fit). Enqueues a
 * fill kernel that zeroes bar and TS, then the launch, both on `stream`;
 * allocates nothing. Every call on a device shares that device's array and
 * finds the previous call's values in S: calls that overlap on one device
 * race, so run them on one stream (or order them). */
int vh_launch_cooperative_noalloc(void* fn, unsigned grid, unsigned block, unsigned dyn_lds, void* stream,
                                  void* const* args, int nargs, int slot, size_t s_bytes, size_t bar_bytes,
                                  size_t ts_bytes);

/* Wait for all work on the current device. */
int vh_synchronize(void);

/* Human-readable text for a status code (static storage). */
const char* vh_error_string(int status);

#ifdef __cplusplus
}
#endif

#endif /* VESTA_HIP_H */
