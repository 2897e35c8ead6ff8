/*
 * A plain C99 client of the backend's C-ABI (include/cchip_runtime.h and
 * include/cchip_backend.h): what any foreign-function binding of
 * libcchip.so does (an OCaml ctypes binding, for one), written in C, so
 * that the headers are shown to be C and the boundary is driven without
 * the Python package. Test infrastructure: __graft_entry__.build() builds
 * it into tests/c_client/libc_client.so and tests/test_c_client.py calls
 * cclient_run through ctypes.
 *
 * The calls follow Backend.S (lib/backend/backend.ml:13-20): compile the
 * graph's wire text, query its params and outputs, run it on host arrays,
 * release it.
 */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "cchip_backend.h"

static size_t dtype_size(int dtype) { return (dtype == 1 || dtype == 3) ? 8 : 4; }

static void set_msg(char *msg, size_t cap, const char *text) {
  if (msg == NULL || cap == 0) return;
  snprintf(msg, cap, "%s", text != NULL ? text : "");
}

/* The byte size of output i of a compiled program (its dtype and shape),
   or 0 where the query fails. */
static size_t output_bytes(const cchip_program *p, int i) {
  const char *name = NULL;
  int dtype = 0, rank = 0, d;
  int64_t dims[8];
  size_t n = 1;
  if (cchip_program_output(p, i, &name, &dtype, &rank, dims) != CCHIP_OK || rank < 0 || rank > 8) return 0;
  for (d = 0; d < rank; d++) n *= (size_t)dims[d];
  return n * dtype_size(dtype);
}

/* Compiles `graph` on device 0 (one stream), checks that it has `n_out`
   outputs whose byte sizes are `out_bytes`, runs it on the named host
   inputs and writes output i into out[i]. Returns the status of the first
   call that fails (CCHIP_INVALID_ARGUMENT, with a message, for a shape
   mismatch found here), and copies cchip_last_error() into `msg`. */
int cclient_run(const char *graph, int n_in, const char *const *names, const void *const *host,
                const size_t *bytes, int n_out, void *const *out, const size_t *out_bytes, char *msg,
                size_t msg_cap) {
  cchip_program *p = NULL;
  int rc, i;
  set_msg(msg, msg_cap, "");
  rc = cchip_backend_compile(graph, 0, 1, &p);
  if (rc != CCHIP_OK) {
    set_msg(msg, msg_cap, cchip_last_error());
    return rc;
  }
  if (cchip_program_num_outputs(p) != n_out) {
    set_msg(msg, msg_cap, "c_client: the program's output count differs from the caller's");
    cchip_program_destroy(p);
    return CCHIP_INVALID_ARGUMENT;
  }
  for (i = 0; i < n_out; i++)
    if (output_bytes(p, i) != out_bytes[i]) {
      set_msg(msg, msg_cap, "c_client: an output's byte size differs from the caller's buffer");
      cchip_program_destroy(p);
      return CCHIP_INVALID_ARGUMENT;
    }
  rc = cchip_program_run(p, n_in, names, host, bytes, out);
  if (rc != CCHIP_OK) set_msg(msg, msg_cap, cchip_last_error());
  i = cchip_program_destroy(p);
  return rc != CCHIP_OK ? rc : i;
}

/* The names of a graph's params, in Graph.params order, written into
   `buf` separated by spaces, without a device (the plan's buffer lines);
   the number of params, or -1. */
int cclient_param_names(const char *graph, char *buf, size_t cap) {
  char *plan = NULL;
  const char *line;
  int n = 0;
  size_t used = 0;
  if (cap == 0 || cchip_backend_plan(graph, &plan) != CCHIP_OK) return -1;
  buf[0] = '\0';
  for (line = plan; line != NULL && *line != '\0';) {
    const char *end = strchr(line, '\n');
    size_t len = end != NULL ? (size_t)(end - line) : strlen(line);
    char name[256], kind[32];
    int idx;
    long long numel;
    char dt[16];
    /* buffer <index> <name> <dtype> <numel> <role> */
    if (len < sizeof name && sscanf(line, "buffer %d %255s %15s %lld %31s", &idx, name, dt, &numel, kind) == 5 &&
        strcmp(kind, "param") == 0 && strncmp(name, "p_", 2) == 0) {
      const size_t k = strlen(name + 2);
      if (used + k + 2 > cap) break;
      if (used > 0) buf[used++] = ' ';
      memcpy(buf + used, name + 2, k);
      used += k;
      buf[used] = '\0';
      n++;
    }
    line = end != NULL ? end + 1 : NULL;
  }
  cchip_free(plan);
  return n;
}
