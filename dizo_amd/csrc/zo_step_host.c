/*
 * zo_step_host.c -- a C99 host of the ZO step through the library's C ABI,
 * with no Python or torch: device memory from hipMalloc, the step from
 * libdizo_amd.so. It is what a non-Python trainer does with the boundary
 * declared in include/dizo_amd.h.
 *
 * Usage: zo_step_host OUT_FILE
 *
 * Three fp16 tensors (70001, 32768 and 5 elements) start from a fixed bit
 * pattern. One ZO step and the first pass of the next one are applied, as the
 * reference's trainer.py:1580-1593 and 1603-1608 order them:
 *   perturb(+1, seed), perturb(-2, seed),
 *   restore + update(seed, g, lr) fused with perturb(+1, seed + 1).
 * Then a projection table over the same tensors, with the starting values as
 * anchors, computes the group norms and applies alpha = 0.75
 * (trainer.py:428-436, 455-457). OUT_FILE receives, in order: the tensors
 * after the ZO passes, the per-group sums of squares before the apply
 * (float64), and the tensors after the apply.
 */
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "dizo_amd.h"

#define NT 3
static const int64_t kNumel[NT] = {70001, 32768, 5};

static int check_dz(int32_t rc, const char* what) {
  if (rc != DZ_OK) {
    fprintf(stderr, "%s failed (%d): %s\n", what, (int)rc, dz_last_error());
    return 1;
  }
  return 0;
}

static int check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    fprintf(stderr, "%s failed: %s\n", what, hipGetErrorString(e));
    return 1;
  }
  return 0;
}

/* Starting bits of element i of tensor t: finite fp16 values of either sign
 * below 2 in magnitude (exponent bit 14 cleared). */
static uint16_t start_bits(int t, int64_t i) {
  const uint32_t h = (uint32_t)i * 2654435761u + (uint32_t)t * 40503u;
  return (uint16_t)((h >> 16) & 0xbfffu);
}

int main(int argc, char** argv) {
  if (argc != 2) {
    fprintf(stderr, "usage: %s OUT_FILE\n", argv[0]);
    return 2;
  }
  const uint64_t seed = 26, seed2 = 27;
  const float eps = 1e-3f, grad = -1.25f, lr = 1e-3f;
  int dev = 0;
  if (check_hip(hipSetDevice(dev), "hipSetDevice")) return 1;

  uint16_t* host[NT];
  void* theta[NT];
  void* anchor[NT];
  uint64_t ptrs[NT], aptrs[NT];
  for (int t = 0; t < NT; ++t) {
    const size_t bytes = (size_t)kNumel[t] * 2;
    host[t] = (uint16_t*)malloc(bytes);
    if (!host[t]) return 1;
    for (int64_t i = 0; i < kNumel[t]; ++i) host[t][i] = start_bits(t, i);
    if (check_hip(hipMalloc(&theta[t], bytes), "hipMalloc") || check_hip(hipMalloc(&anchor[t], bytes), "hipMalloc"))
      return 1;
    if (check_hip(hipMemcpy(theta[t], host[t], bytes, hipMemcpyHostToDevice), "hipMemcpy") ||
        check_hip(hipMemcpy(anchor[t], host[t], bytes, hipMemcpyHostToDevice), "hipMemcpy"))
      return 1;
    ptrs[t] = (uint64_t)(uintptr_t)theta[t];
    aptrs[t] = (uint64_t)(uintptr_t)anchor[t];
  }

  /* A ZO table: NULL z offsets lay the tensors end to end. */
  dz_table* zo = NULL;
  if (check_dz(dz_table_create(ptrs, NULL, kNumel, NULL, NT, DZ_DTYPE_F16, dev, &zo), "dz_table_create")) return 1;
  if (check_dz(dz_perturb(zo, seed, 1.0f, eps, NULL, NULL), "dz_perturb(+1)") ||
      check_dz(dz_perturb(zo, seed, -2.0f, eps, NULL, NULL), "dz_perturb(-2)") ||
      check_dz(dz_restore_update_perturb(zo, seed, seed2, eps, grad, lr, NULL, NULL, NULL, NULL, NULL),
               "dz_restore_update_perturb"))
    return 1;
  /* An invalid call returns an error code and leaves a message; nothing aborts. */
  if (dz_perturb(NULL, seed, 1.0f, eps, NULL, NULL) >= 0 || dz_last_error()[0] == '\0') {
    fprintf(stderr, "a NULL table was not rejected\n");
    return 1;
  }

  FILE* out = fopen(argv[1], "wb");
  if (!out) return 1;
  if (check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize")) return 1;
  for (int t = 0; t < NT; ++t) {
    const size_t bytes = (size_t)kNumel[t] * 2;
    if (check_hip(hipMemcpy(host[t], theta[t], bytes, hipMemcpyDeviceToHost), "hipMemcpy")) return 1;
    fwrite(host[t], 1, bytes, out);
  }

  /* A projection table over the same tensors, anchored at the starting values. */
  dz_table* proj = NULL;
  double* d_sumsq = NULL;
  uint16_t* d_alpha = NULL;
  const uint16_t alpha_bits[NT] = {0x3a00, 0x3a00, 0x3a00}; /* 0.75 in fp16 */
  double sumsq[NT];
  if (check_dz(dz_table_create(ptrs, aptrs, kNumel, NULL, NT, DZ_DTYPE_F16, dev, &proj), "dz_table_create(proj)"))
    return 1;
  if (check_hip(hipMalloc((void**)&d_sumsq, sizeof(sumsq)), "hipMalloc") ||
      check_hip(hipMalloc((void**)&d_alpha, sizeof(alpha_bits)), "hipMalloc") ||
      check_hip(hipMemcpy(d_alpha, alpha_bits, sizeof(alpha_bits), hipMemcpyHostToDevice), "hipMemcpy"))
    return 1;
  if (check_dz(dz_group_sumsq(proj, d_sumsq, NULL, NULL, NULL), "dz_group_sumsq") ||
      check_dz(dz_project(proj, d_alpha, DZ_PROJ_APPLY, NULL, NULL, NULL, NULL), "dz_project(apply)"))
    return 1;
  if (check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize") ||
      check_hip(hipMemcpy(sumsq, d_sumsq, sizeof(sumsq), hipMemcpyDeviceToHost), "hipMemcpy"))
    return 1;
  fwrite(sumsq, sizeof(double), NT, out);
  for (int t = 0; t < NT; ++t) {
    const size_t bytes = (size_t)kNumel[t] * 2;
    if (check_hip(hipMemcpy(host[t], theta[t], bytes, hipMemcpyDeviceToHost), "hipMemcpy")) return 1;
    fwrite(host[t], 1, bytes, out);
  }
  fclose(out);

  if (check_dz(dz_table_destroy(zo), "dz_table_destroy") || check_dz(dz_table_destroy(proj), "dz_table_destroy"))
    return 1;
  for (int t = 0; t < NT; ++t) {
    (void)hipFree(theta[t]);
    (void)hipFree(anchor[t]);
    free(host[t]);
  }
  (void)hipFree(d_sumsq);
  (void)hipFree(d_alpha);
  printf("zo_step_host ok\n");
  return 0;
}
