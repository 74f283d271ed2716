/*
 * abi_check.c: drives libvllm_rlt_hip.so through include/vllm_rlt_hip.h from
 * plain C (no Python, no torch): the C caller a maintainer's cgo / JNI /
 * native binding would be. On one GPU it
 *   1. checks the ABI version;
 *   2. appends one token per row (vrh_kv_append) and reads the pool back;
 *   3. runs split-KV decode (vrh_paged_decode, caller workspace) over a
 *      grouped-query f32 batch with a zero-length row and compares every
 *      output with a double-precision host computation of the reference
 *      semantics (kernels/paged_attention.py:12-36);
 *   4. runs vrh_paged_decode_noalloc on the same inputs: bit-identical;
 *   5. checks the error path (unknown dtype: VRH_ERROR_INVALID_ARG and a
 *      message from vrh_last_error()).
 * Prints "abi_check: OK" and exits 0, or names the failing check and exits 1.
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "vllm_rlt_hip.h"

enum { BLOCKS = 40, BS = 16, KVH = 2, QH = 4, D = 64, ROWS = 3, WIDTH = 20 };

static int fail(const char* what) {
  printf("abi_check: FAILED: %s\n", what);
  return 1;
}

#define HIP_OK(call)                                        \
  do {                                                      \
    if ((call) != hipSuccess) return fail(#call);           \
  } while (0)

static uint32_t lcg_state = 12345u;
static float rnd(void) {
  lcg_state = lcg_state * 1664525u + 1013904223u;
  return ((float)(lcg_state >> 8) / 16777216.0f) * 2.0f - 1.0f;
}

int main(void) {
  const int lengths[ROWS] = {0, 17, 300};
  const size_t slot = (size_t)KVH * D;                 /* floats per token slot */
  const size_t pool_floats = (size_t)BLOCKS * BS * slot;
  float* hk = malloc(pool_floats * sizeof(float));
  float* hv = malloc(pool_floats * sizeof(float));
  float* hq = malloc((size_t)ROWS * QH * D * sizeof(float));
  float* knew = malloc((size_t)ROWS * slot * sizeof(float));
  float* vnew = malloc((size_t)ROWS * slot * sizeof(float));
  float* out = malloc((size_t)ROWS * QH * D * sizeof(float));
  float* out2 = malloc((size_t)ROWS * QH * D * sizeof(float));
  int32_t tables[ROWS * WIDTH];
  int64_t wblocks[ROWS], woffs[ROWS];
  if (!hk || !hv || !hq || !knew || !vnew || !out || !out2) return fail("host allocation");

  if (vrh_abi_version() != 5) return fail("vrh_abi_version() != 5");
  for (size_t i = 0; i < pool_floats; ++i) {
    hk[i] = rnd();
    hv[i] = rnd();
  }
  for (int i = 0; i < ROWS * QH * D; ++i) hq[i] = rnd();
  for (size_t i = 0; i < ROWS * slot; ++i) {
    knew[i] = rnd();
    vnew[i] = rnd();
  }
  /* Tables: distinct pages in a scrambled order; -1 past each row's pages. */
  int next = 0;
  for (int r = 0; r < ROWS; ++r)
    for (int p = 0; p < WIDTH; ++p) {
      const int pages = (lengths[r] + BS - 1) / BS;
      tables[r * WIDTH + p] = p < pages ? (next++ * 7) % BLOCKS : -1;
    }
  /* Row r appends its last token (position lengths[r] - 1); row 0 is
   * disabled through the mask. */
  uint8_t mask[ROWS] = {0, 1, 1};
  for (int r = 0; r < ROWS; ++r) {
    const int pos = lengths[r] > 0 ? lengths[r] - 1 : 0;
    wblocks[r] = tables[r * WIDTH + pos / BS] < 0 ? 0 : tables[r * WIDTH + pos / BS];
    woffs[r] = pos % BS;
  }

  float *dk, *dv, *dq, *dknew, *dvnew, *dout, *dout2;
  int32_t *dtab, *dlen;
  int64_t *dwb, *dwo;
  uint8_t* dmask;
  void* ws;
  const size_t ws_bytes = vrh_paged_decode_workspace_bytes(ROWS, QH, D);
  HIP_OK(hipMalloc((void**)&dk, pool_floats * sizeof(float)));
  HIP_OK(hipMalloc((void**)&dv, pool_floats * sizeof(float)));
  HIP_OK(hipMalloc((void**)&dq, (size_t)ROWS * QH * D * sizeof(float)));
  HIP_OK(hipMalloc((void**)&dknew, ROWS * slot * sizeof(float)));
  HIP_OK(hipMalloc((void**)&dvnew, ROWS * slot * sizeof(float)));
  HIP_OK(hipMalloc((void**)&dout, (size_t)ROWS * QH * D * sizeof(float)));
  HIP_OK(hipMalloc((void**)&dout2, (size_t)ROWS * QH * D * sizeof(float)));
  HIP_OK(hipMalloc((void**)&dtab, sizeof(tables)));
  HIP_OK(hipMalloc((void**)&dlen, sizeof(lengths)));
  HIP_OK(hipMalloc((void**)&dwb, sizeof(wblocks)));
  HIP_OK(hipMalloc((void**)&dwo, sizeof(woffs)));
  HIP_OK(hipMalloc((void**)&dmask, sizeof(mask)));
  HIP_OK(hipMalloc(&ws, ws_bytes));
  HIP_OK(hipMemcpy(dk, hk, pool_floats * sizeof(float), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dv, hv, pool_floats * sizeof(float), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dq, hq, (size_t)ROWS * QH * D * sizeof(float), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dknew, knew, ROWS * slot * sizeof(float), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dvnew, vnew, ROWS * slot * sizeof(float), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dtab, tables, sizeof(tables), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dlen, lengths, sizeof(lengths), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dwb, wblocks, sizeof(wblocks), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dwo, woffs, sizeof(woffs), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dmask, mask, sizeof(mask), hipMemcpyHostToDevice));

  /* 2. append (one layer view: block stride BS*slot, token stride slot). */
  if (vrh_kv_append(VRH_DTYPE_F32, dk, dv, BS * slot, slot, D, 0, dknew, dvnew, slot, D, 0, slot,
                    D, 0, dwb, dwo, dmask, NULL, ROWS, 1, KVH, D, BLOCKS, BS, 0) != VRH_OK)
    return fail(vrh_last_error());
  for (int r = 0; r < ROWS; ++r) {
    if (!mask[r]) continue;
    float* dst_k = hk + (size_t)(wblocks[r] * BS + woffs[r]) * slot;
    float* dst_v = hv + (size_t)(wblocks[r] * BS + woffs[r]) * slot;
    memcpy(dst_k, knew + r * slot, slot * sizeof(float));
    memcpy(dst_v, vnew + r * slot, slot * sizeof(float));
  }
  float* back = malloc(pool_floats * sizeof(float));
  if (!back) return fail("host allocation");
  HIP_OK(hipMemcpy(back, dk, pool_floats * sizeof(float), hipMemcpyDeviceToHost));
  if (memcmp(back, hk, pool_floats * sizeof(float)) != 0) return fail("append: K pool differs");
  HIP_OK(hipMemcpy(back, dv, pool_floats * sizeof(float), hipMemcpyDeviceToHost));
  if (memcmp(back, hv, pool_floats * sizeof(float)) != 0) return fail("append: V pool differs");

  /* 3. decode with a caller workspace. */
  if (vrh_paged_decode(VRH_DTYPE_F32, dout, dq, dk, dv, dtab, dlen, ROWS, QH, KVH, D, BS, WIDTH,
                       WIDTH, QH * D, D, QH * D, D, BS * slot, slot, D, BS * slot, slot, D, 0, ws,
                       ws_bytes, 0) != VRH_OK)
    return fail(vrh_last_error());
  HIP_OK(hipMemcpy(out, dout, (size_t)ROWS * QH * D * sizeof(float), hipMemcpyDeviceToHost));
  double max_err = 0.0;
  for (int r = 0; r < ROWS; ++r)
    for (int h = 0; h < QH; ++h) {
      const int kvh = h / (QH / KVH);
      const float* q = hq + ((size_t)r * QH + h) * D;
      const int n = lengths[r];
      double m = -INFINITY, l = 0.0, acc[D];
      for (int d = 0; d < D; ++d) acc[d] = 0.0;
      double* s = malloc((size_t)(n > 0 ? n : 1) * sizeof(double));
      if (!s) return fail("host allocation");
      for (int t = 0; t < n; ++t) {
        const float* k = hk + ((size_t)tables[r * WIDTH + t / BS] * BS + t % BS) * slot + kvh * D;
        double dot = 0.0;
        for (int d = 0; d < D; ++d) dot += (double)q[d] * k[d];
        s[t] = dot / sqrt((double)D);
        if (s[t] > m) m = s[t];
      }
      for (int t = 0; t < n; ++t) {
        const float* v = hv + ((size_t)tables[r * WIDTH + t / BS] * BS + t % BS) * slot + kvh * D;
        const double p = exp(s[t] - m);
        l += p;
        for (int d = 0; d < D; ++d) acc[d] += p * v[d];
      }
      free(s);
      for (int d = 0; d < D; ++d) {
        const double want = n > 0 ? acc[d] / l : 0.0;
        const double err = fabs(want - out[((size_t)r * QH + h) * D + d]);
        if (err > max_err) max_err = err;
      }
    }
  if (!(max_err <= 1e-4)) {
    printf("abi_check: decode max abs error %g\n", max_err);
    return fail("decode differs from the host computation");
  }

  /* 4. the allocation-free entry point gives the same bits. */
  if (vrh_paged_decode_noalloc(VRH_DTYPE_F32, dout2, dq, dk, dv, dtab, dlen, ROWS, QH, KVH, D, BS,
                               WIDTH, WIDTH, QH * D, D, QH * D, D, BS * slot, slot, D, BS * slot,
                               slot, D, 0, 0) != VRH_OK)
    return fail(vrh_last_error());
  HIP_OK(hipMemcpy(out2, dout2, (size_t)ROWS * QH * D * sizeof(float), hipMemcpyDeviceToHost));
  if (memcmp(out, out2, (size_t)ROWS * QH * D * sizeof(float)) != 0)
    return fail("noalloc decode differs from the workspace decode");

  /* 5. error path: an unknown dtype is refused before any launch. */
  if (vrh_paged_decode(99, dout, dq, dk, dv, dtab, dlen, ROWS, QH, KVH, D, BS, WIDTH, WIDTH,
                       QH * D, D, QH * D, D, BS * slot, slot, D, BS * slot, slot, D, 0, ws,
                       ws_bytes, 0) != VRH_ERROR_INVALID_ARG)
    return fail("unknown dtype accepted");
  if (strlen(vrh_last_error()) == 0) return fail("no error message");

  HIP_OK(hipDeviceSynchronize());
  printf("abi_check: decode max abs error %.3g\n", max_err);
  printf("abi_check: OK\n");
  return 0;
}
