/*
 * cchip backend: Backend_hip, the gfx950 execution backend behind the
 * reference's plugin signature Backend.S (lib/backend/backend.ml:13-20) and
 * the extensions Backend_cuda adds (lib/backend_cuda/cudacaml_backend_cuda.mli
 * :7-84), as a C-ABI.
 *
 * A graph crosses the boundary as the text wire format "cchip-graph 1"
 * (cudacaml_amd/ir.py writes it; an OCaml caller prints the same text from
 * a Graph.t): one line per expression node ("x"), per tensor node in
 * topological order ("t"), per output ("o"), then "end". compile runs the
 * fusion plan, instantiates the CDNA4
 * kernel templates, JITs them with hiprtc and allocates the executor pools;
 * run walks the host plan (upload, launch, download) on the executor's
 * stream.
 *
 * Status codes and cchip_last_error() are those of cchip_runtime.h.
 * Host inputs and outputs are raw row-major element data; their dtype and
 * shape are the program's (query them with cchip_program_param/output).
 * Dtype codes: 0 f32, 1 f64, 2 i32, 3 i64.
 */
#ifndef CCHIP_BACKEND_H
#define CCHIP_BACKEND_H

#include <stddef.h>
#include <stdint.h>

#include "cchip_runtime.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct cchip_program cchip_program;
typedef struct cchip_job cchip_job;

/* The generated HIP source for a graph, without compiling it
   (Backend_cuda.source). Free the string with cchip_free. */
int cchip_backend_source(const char *graph, char **source);
/* The kernel list and host plan as text, one op per line, without a device
   (the introspection Lower.program gives the reference's tests). */
int cchip_backend_plan(const char *graph, char **plan);
void cchip_free(void *p);

/* Backend.S.compile / compile_with ~streams / compile_on ~device:
   JIT once, then `streams` executors, each with its own stream and buffer
   pool; executor 0 uses the NULL stream (cudacaml_backend_cuda.ml:326-339). */
int cchip_backend_compile(const char *graph, int device, int streams, cchip_program **program);
/* Frees every device buffer. Idempotent; a run afterwards fails
   (Backend_cuda.release). */
int cchip_program_release(cchip_program *program);
/* release plus freeing the handle itself. */
int cchip_program_destroy(cchip_program *program);

int cchip_program_device(const cchip_program *program);
int cchip_program_streams(const cchip_program *program);
/* Device allocations executor 0 holds (Executor.buffer_count): one per
   buffer of the plan, except that params and outputs of at most 4 KiB and
   the error word share a single one. */
int cchip_program_buffer_count(const cchip_program *program);
int cchip_program_kernel_count(const cchip_program *program);
const char *cchip_program_kernel_name(const cchip_program *program, int i);

int cchip_program_num_params(const cchip_program *program);
/* Name, dtype, rank and dims (up to 8) of param i, in Graph.params order. */
int cchip_program_param(const cchip_program *program, int i, const char **name, int *dtype, int *rank,
                        int64_t *dims);
int cchip_program_num_outputs(const cchip_program *program);
int cchip_program_output(const cchip_program *program, int i, const char **name, int *dtype, int *rank,
                         int64_t *dims);

/* Backend.S.run: synchronous, executor 0. Inputs are matched to params by
   name and must have exactly the param's byte size (CCHIP_INVALID_ARGUMENT
   otherwise, before any device work). `outputs[i]` receives output i in
   Graph.outputs order. A device-side index error (gather or scatter_add
   out of range) is CCHIP_INVALID_ARGUMENT after the run. */
int cchip_program_run(cchip_program *program, int n_inputs, const char *const *names, const void *const *host,
                      const size_t *bytes, void *const *outputs);

/* run_async / wait: issue on the next executor of the ring and return; the
   host input and output memory must stay valid until cchip_job_wait
   returns. wait may be called more than once (cudacaml_backend_cuda.ml
   :357-365). Each job reports only the device-side index errors of its own
   run (and of run_resident_into calls with sync == 0 queued on its lane
   before it): its lane's stream copies the error word into the job's own
   pinned slot and then clears it. */
int cchip_program_run_async(cchip_program *program, int n_inputs, const char *const *names,
                            const void *const *host, const size_t *bytes, void *const *outputs, cchip_job **job);
int cchip_job_wait(cchip_job *job);
int cchip_job_free(cchip_job *job);

/* run_resident: device in, device out (executor.ml:181-244). Input device
   buffers replace the param buffers by name (no copy); each output gets a
   fresh device buffer in `outputs[i]` that the caller frees with
   cchip_buffer_free. Synchronises before returning. */
int cchip_program_run_resident(cchip_program *program, int n_inputs, const char *const *names,
                               void *const *dev_inputs, const size_t *bytes, void **outputs);

/* Extension for serving loops and benchmarks, no reference counterpart:
   like run_resident but the caller supplies the output device buffers
   (exact byte sizes) and chooses whether to synchronise. With sync == 0
   the call only issues work on executor 0's stream; device-side index
   errors are then reported by the next synchronising call. */
int cchip_program_run_resident_into(cchip_program *program, int n_inputs, const char *const *names,
                                    void *const *dev_inputs, const size_t *bytes, void *const *dev_outputs,
                                    int sync);

/* No counterpart in the reference. For callers that cannot allocate device
   memory: code under HIP graph capture, serving loops, harnesses that
   forbid hipMalloc. Runs like run_resident_into with sync == 0, but on
   `stream` (NULL: the default stream), and calls no hipMalloc, hipFree or
   other allocating routine. The template scratch (look-back status words,
   split partials, scatter counts and staged pairs) comes from a static
   device array of 32 MiB per GPU inside this library instead of the
   program's pool; it is cleared by a kernel at the start of every call.
   A program whose scratch exceeds 32 MiB is CCHIP_INVALID_ARGUMENT before
   any device work. All calls on one GPU share that array, and each uses the
   program's executor-0 pool for its intermediates: calls that overlap on
   one GPU (any program), or that overlap another run of the same program,
   race. Device-side index errors stay with the call: its error word is the
   first word of the static scratch, cleared at the start of the call, and
   never the program's own, so no other run reports them. When `err_out` (a
   device int the caller owns) is not NULL, the call copies its word there
   after its kernels, on `stream`; 0 means no error, and
   cchip_error_word_status turns any other value into the status and
   message a synchronous run would have given. With `err_out` NULL the
   flags are dropped. Work is only issued; synchronise `stream` before
   reading the outputs or `err_out`. */
int cchip_program_run_resident_noalloc(cchip_program *program, int n_inputs, const char *const *names,
                                       void *const *dev_inputs, const size_t *bytes, void *const *dev_outputs,
                                       void *stream, int *err_out);
/* No counterpart in the reference; the companion of the allocation-free
   run. CCHIP_OK for 0; otherwise CCHIP_INVALID_ARGUMENT with
   cchip_last_error() set to the interpreter's message for the device-side
   error flags in `code` (gather or scatter_add index out of bounds, or a
   look-back scan that did not complete). */
int cchip_error_word_status(int code);

/* The stream executor `lane` issues its work on (NULL for lane 0). */
int cchip_program_stream(const cchip_program *program, int lane, void **stream);

/* Timing hook for measurement: while enabled, executor 0 records a pair of
   timing events around every launch of kernel `name`; cchip_program_timing
   returns the number of such launches since enabling and their summed
   device time. Synchronise the stream before reading. */
int cchip_program_time_kernel(cchip_program *program, const char *name);
int cchip_program_timing(cchip_program *program, int *launches, double *total_ms);
/* As cchip_program_timing, also writing the first `capacity` per-launch
   durations (ms, launch order) to `each_ms`. */
int cchip_program_timing_each(cchip_program *program, int capacity, double *each_ms, int *launches,
                              double *total_ms);

#ifdef __cplusplus
}
#endif

#endif
