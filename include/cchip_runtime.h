/*
 * cchip runtime: the C-ABI that replaces CUDACaml's lib/runtime (which sits
 * on cudajit -> libcuda + libnvrtc) with one over the HIP module API and
 * hiprtc, for gfx950 only. One function per value of the OCaml runtime
 * interface; an OCaml `lib/runtime` rewrite binds these with ctypes.
 * Plain pointers and sizes only.
 *
 * Every function that can fail returns a status:
 *   CCHIP_OK (0), CCHIP_INVALID_ARGUMENT (1) for caller mistakes (the
 *   reference raises Invalid_argument), CCHIP_FAILURE (2) for driver, JIT
 *   and plan errors (the reference raises Failure). The message of the last
 *   failure on the calling thread is cchip_last_error().
 */
#ifndef CCHIP_RUNTIME_H
#define CCHIP_RUNTIME_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CCHIP_OK 0
#define CCHIP_INVALID_ARGUMENT 1
#define CCHIP_FAILURE 2

/* Message of the last non-OK status returned on this thread. */
const char *cchip_last_error(void);

/* ---- Device: lib/runtime/device.mli:3-57 -------------------------------- */

/* 1 when a HIP device is usable, else 0. Never fails and never prints
   (replaces Device.available, device.ml:44-53). */
int cchip_device_available(void);
/* Idempotent runtime initialisation on device 0 (Device.init). */
int cchip_device_init(void);
/* Blocks until all work on the current device is done (Device.synchronize). */
int cchip_device_synchronize(void);
/* Number of devices the runtime reports (Device.count). */
int cchip_device_count(int *count);
/* Current device ordinal of the calling thread (Device.current). */
int cchip_device_get(int *ordinal);
/* Make `ordinal` current on the calling thread; Device.with_device is built
   on get/set by the host language so it can restore on exceptions. */
int cchip_device_set(int ordinal);
/* Device.info_of: name, architecture ("gfx950"), compute units, HBM bytes.
   The architecture string replaces the reference's (major, minor) pair:
   Device.info_to_string prints "compute: gfx950" where CUDA printed
   "compute: sm_XY". */
int cchip_device_info(int ordinal, char *name, size_t name_len, char *arch, size_t arch_len,
                      int *multiprocessors, int64_t *total_memory_bytes);

/* ---- Buffer: lib/runtime/buffer.mli:6-31 ------------------------------- */

/* Device allocation on the current device. A 0-byte request allocates one
   byte so every buffer is a distinct, valid pointer (buffer.ml:14-20). */
int cchip_buffer_alloc(size_t bytes, void **dptr);
int cchip_buffer_free(void *dptr);
/* Allocations minus frees since process start (Buffer.live_count). */
int64_t cchip_buffer_live_count(void);
/* Synchronous copies (Buffer.upload / Buffer.download). */
int cchip_buffer_upload(void *dst, const void *src, size_t bytes);
int cchip_buffer_download(void *dst, const void *src, size_t bytes);
/* Stream-ordered copies; the host memory must stay valid until the stream
   has been synchronised (Buffer.upload_async / download_async). */
int cchip_buffer_upload_async(void *dst, const void *src, size_t bytes, void *stream);
int cchip_buffer_download_async(void *dst, const void *src, size_t bytes, void *stream);
/* Device-to-device, stream-ordered (Buffer.copy_device). */
int cchip_buffer_copy_device(void *dst, const void *src, size_t bytes, void *stream);

/* ---- Stream: lib/runtime/stream.mli:9-36 ------------------------------- */

/* The NULL stream is the default stream (Stream.default). create makes a
   non-blocking stream at the default priority (Stream.create). */
int cchip_stream_create(void **stream);
int cchip_stream_destroy(void *stream);
int cchip_stream_synchronize(void *stream);
/* *idle = 1 when every operation issued on the stream has completed. */
int cchip_stream_is_idle(void *stream, int *idle);

/* ---- Event: lib/runtime/event.mli:4-20 --------------------------------- */

/* Creates a timing-enabled event and records it on `stream` (Event.record). */
int cchip_event_record(void *stream, void **event);
/* Work issued on `stream` after this waits for `event` (Event.wait). */
int cchip_event_wait(void *stream, void *event);
int cchip_event_synchronize(void *event);
/* Milliseconds between two completed events (Event.elapsed_ms). */
int cchip_event_elapsed_ms(void *start, void *stop, float *ms);
int cchip_event_destroy(void *event);

/* ---- Jit: lib/runtime/jit.mli:6-17 ------------------------------------- */

/* hiprtc (--offload-arch=gfx950) then hipModuleLoadData. A compile error
   is CCHIP_FAILURE with the hiprtc log in cchip_last_error(), never
   swallowed (jit.ml:11-25). Code objects are cached by source hash. */
int cchip_jit_compile(const char *name, const char *source, void **module);
/* Compile only, no device needed: the code object's size (the HIP
   counterpart of Jit.ptx, which has no textual PTX). */
int cchip_jit_check(const char *name, const char *source, size_t *code_bytes);
int cchip_jit_code_size(void *module, size_t *bytes);
/* Kernel handle by name; CCHIP_FAILURE on an unknown name (jit.ml:29-30). */
int cchip_jit_get_kernel(void *module, const char *name, void **kernel);
int cchip_jit_unload(void *module);

/* ---- Launch: lib/runtime/launch.mli:7-16 ------------------------------- */

/* Asynchronous launch. Arguments are device pointers only; every scalar is
   baked into the source (launch.mli:1-2). */
int cchip_launch(void *kernel, int grid, int grid_y, int block, int block_y, int shared_bytes, void *stream,
                 int nargs, void *const *dev_ptrs);

/* ---- Pinned: lib/runtime/pinned.mli:17-33 ------------------------------ */

/* Portable page-locked host memory, zero-filled (Pinned.alloc). */
int cchip_pinned_alloc(size_t bytes, void **host);
int cchip_pinned_free(void *host);
/* 1 if `host` is the start of a live cchip_pinned_alloc block (Pinned.is_pinned). */
int cchip_pinned_is_pinned(const void *host);

#ifdef __cplusplus
}
#endif

#endif
