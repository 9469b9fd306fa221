/*
 * fagq_c_check.c - the operator called from a plain C host through the C ABI
 * (include/fagq.h), with no Python or torch in the process: the drop-in
 * boundary as a C or C++ caller of the reference's operator would use it.
 *
 *   fagq_c_check M D DIR
 *
 * reads DIR/x.bin, DIR/residual.bin ([M, D] bf16) and DIR/gamma.bin ([D]
 * bf16), runs fagq_launch (fp8 e4m3fn codes, fp32 column-major scales, group
 * 128, eps 1e-6, norm_out written) on the default stream, and writes
 * DIR/residual_out.bin, DIR/norm_out.bin, DIR/q.bin and DIR/scale.bin
 * ([D / 128, M] fp32).  It then checks that fagq_launch rejects a NULL
 * pointer and a bad group size before any device work.  Exit status 0 on
 * success; any failure prints the status and exits 1.
 */
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "fagq.h"

static int read_file(const char* dir, const char* name, void* buf, size_t n) {
  char path[4096];
  snprintf(path, sizeof path, "%s/%s", dir, name);
  FILE* f = fopen(path, "rb");
  if (!f) return -1;
  const size_t got = fread(buf, 1, n, f);
  fclose(f);
  return got == n ? 0 : -1;
}

static int write_file(const char* dir, const char* name, const void* buf, size_t n) {
  char path[4096];
  snprintf(path, sizeof path, "%s/%s", dir, name);
  FILE* f = fopen(path, "wb");
  if (!f) return -1;
  const size_t put = fwrite(buf, 1, n, f);
  fclose(f);
  return put == n ? 0 : -1;
}

#define HIP_OK(call)                                                          \
  do {                                                                        \
    hipError_t e_ = (call);                                                   \
    if (e_ != hipSuccess) {                                                   \
      fprintf(stderr, "%s: %s\n", #call, hipGetErrorString(e_));              \
      return 1;                                                               \
    }                                                                         \
  } while (0)

int main(int argc, char** argv) {
  if (argc != 4) {
    fprintf(stderr, "usage: %s M D DIR\n", argv[0]);
    return 1;
  }
  const int64_t M = atoll(argv[1]), D = atoll(argv[2]), G = 128;
  const char* dir = argv[3];
  if (M <= 0 || D <= 0 || D % G != 0) {
    fprintf(stderr, "bad shape\n");
    return 1;
  }
  const size_t ne = (size_t)(M * D), nsc = (size_t)(M * (D / G));
  uint16_t* hx = malloc(ne * 2);
  uint16_t* hr = malloc(ne * 2);
  uint16_t* hg = malloc((size_t)D * 2);
  uint16_t* hro = malloc(ne * 2);
  uint16_t* hno = malloc(ne * 2);
  uint8_t* hq = malloc(ne);
  float* hs = malloc(nsc * 4);
  if (!hx || !hr || !hg || !hro || !hno || !hq || !hs) return 1;
  if (read_file(dir, "x.bin", hx, ne * 2) || read_file(dir, "residual.bin", hr, ne * 2) ||
      read_file(dir, "gamma.bin", hg, (size_t)D * 2)) {
    fprintf(stderr, "cannot read the inputs in %s\n", dir);
    return 1;
  }

  void *x, *r, *g, *ro, *no, *q, *s;
  HIP_OK(hipMalloc(&x, ne * 2));
  HIP_OK(hipMalloc(&r, ne * 2));
  HIP_OK(hipMalloc(&g, (size_t)D * 2));
  HIP_OK(hipMalloc(&ro, ne * 2));
  HIP_OK(hipMalloc(&no, ne * 2));
  HIP_OK(hipMalloc(&q, ne));
  HIP_OK(hipMalloc(&s, nsc * 4));
  HIP_OK(hipMemcpy(x, hx, ne * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(r, hr, ne * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(g, hg, (size_t)D * 2, hipMemcpyHostToDevice));

  int st = fagq_launch(x, r, g, ro, no, q, s, M, D, G, 1e-6f, FAGQ_Q_FP8_E4M3FN, FAGQ_SCALE_F32,
                       FAGQ_LAYOUT_COL_MAJOR, FAGQ_ROUND_RNE, NULL);
  if (st != FAGQ_OK) {
    fprintf(stderr, "fagq_launch: %d (%s)\n", st, fagq_status_string(st));
    return 1;
  }
  HIP_OK(hipDeviceSynchronize());
  HIP_OK(hipMemcpy(hro, ro, ne * 2, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(hno, no, ne * 2, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(hq, q, ne, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(hs, s, nsc * 4, hipMemcpyDeviceToHost));
  if (write_file(dir, "residual_out.bin", hro, ne * 2) || write_file(dir, "norm_out.bin", hno, ne * 2) ||
      write_file(dir, "q.bin", hq, ne) || write_file(dir, "scale.bin", hs, nsc * 4)) {
    fprintf(stderr, "cannot write the outputs in %s\n", dir);
    return 1;
  }

  /* Argument errors come back as status codes, before any device work. */
  st = fagq_launch(NULL, r, g, ro, no, q, s, M, D, G, 1e-6f, FAGQ_Q_FP8_E4M3FN, FAGQ_SCALE_F32,
                   FAGQ_LAYOUT_COL_MAJOR, FAGQ_ROUND_RNE, NULL);
  if (st != FAGQ_E_NULL) {
    fprintf(stderr, "NULL x: expected FAGQ_E_NULL, got %d\n", st);
    return 1;
  }
  st = fagq_launch(x, r, g, ro, no, q, s, M, D, 100, 1e-6f, FAGQ_Q_FP8_E4M3FN, FAGQ_SCALE_F32,
                   FAGQ_LAYOUT_COL_MAJOR, FAGQ_ROUND_RNE, NULL);
  if (st != FAGQ_E_GROUP) {
    fprintf(stderr, "group 100: expected FAGQ_E_GROUP, got %d\n", st);
    return 1;
  }

  hipFree(x);
  hipFree(r);
  hipFree(g);
  hipFree(ro);
  hipFree(no);
  hipFree(q);
  hipFree(s);
  free(hx);
  free(hr);
  free(hg);
  free(hro);
  free(hno);
  free(hq);
  free(hs);
  printf("fagq_c_check: ok (libfagq version %d)\n", fagq_version());
  return 0;
}
