/*
 * oracle_simd.c -- multi-threaded, vectorised restatement of woolly's intended
 * x86 SIMD quantized GEMV, for the CPU baseline of the benchmark.
 *
 * TEST INFRASTRUCTURE ONLY: bench.py times it as the CPU baseline and the CPU
 * tests check it; the product (woolly_amd, libwoolly_hip.so) never links,
 * loads or calls it.
 *
 * Follows qmatvec_q4_0_avx2 / qmatvec_q8_0_avx2
 * (crates/woolly-tensor/src/quantization.rs:720-840): per row one 8-lane f32
 * accumulator; per block the scale d; per 8-element chunk the weights
 * w = q * d - 8 d (Q4_0, one fused multiply-add, :757) or w = q * d (Q8_0,
 * :813), then sum = fma(w, x, sum) (:760, :816); a horizontal sum of the 8 lanes
 * at the end of the row (:765-773).  The reference's Q4_0 kernel takes the low
 * nibble of qs[4c .. 4c+7] for chunk c (:750-753), which reads the wrong
 * elements; here chunks 0-1 take the low nibbles of qs[0..15] (elements 0-15)
 * and chunks 2-3 the high nibbles (elements 16-31), the element order of
 * dequantize_q4_0 (:473-481).  Q4_1 has no SIMD kernel in the reference; it is
 * w = q * d + m (dequantize_q4_1, :500-506) in the same loop.
 *
 * Rows are split into contiguous ranges over POSIX threads.  Built with
 * -O3 -mavx2 -mfma so the 8-lane loops compile to ymm FMAs;
 * orc_simd_available() says whether this CPU can run it.
 */
#include <math.h>
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>

#include "oracle.h"

typedef struct {
  int type;
  const uint8_t* w;
  const float* x;
  float* y;
  size_t r0, r1, k;
} job_t;

static float h2f(const uint8_t* p) { return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

static void rows(const job_t* j) {
  const size_t nb = j->k / 32, ts = orc_type_size(j->type);
  for (size_t row = j->r0; row < j->r1; row++) {
    float sum[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const uint8_t* rp = j->w + row * nb * ts;
    for (size_t b = 0; b < nb; b++) {
      const uint8_t* blk = rp + b * ts;
      const float* in = j->x + b * 32;
      const float d = h2f(blk);
      for (int c = 0; c < 4; c++) {
        float q[8], wv[8];
        if (j->type == ORC_Q8_0) {
          const int8_t* qs = (const int8_t*)(blk + 2) + 8 * c;
          for (int l = 0; l < 8; l++) q[l] = (float)qs[l];
          for (int l = 0; l < 8; l++) wv[l] = q[l] * d;
        } else {
          const uint8_t* qs = blk + (j->type == ORC_Q4_1 ? 4 : 2) + 8 * (c & 1);
          const int shift = c < 2 ? 0 : 4;
          for (int l = 0; l < 8; l++) q[l] = (float)((qs[l] >> shift) & 0x0F);
          if (j->type == ORC_Q4_0) {
            const float off = -8.0f * d;
            for (int l = 0; l < 8; l++) wv[l] = fmaf(q[l], d, off);
          } else {
            const float m = h2f(blk + 2);
            for (int l = 0; l < 8; l++) wv[l] = fmaf(q[l], d, m);
          }
        }
        for (int l = 0; l < 8; l++) sum[l] = fmaf(wv[l], in[8 * c + l], sum[l]);
      }
    }
    /* horizontal sum in the reference's order: (hi + lo) then pairwise */
    float s4[4];
    for (int l = 0; l < 4; l++) s4[l] = sum[l + 4] + sum[l];
    const float s0 = s4[0] + s4[1], s2 = s4[2] + s4[3];
    j->y[row] = s0 + s2;
  }
}

static void* worker(void* arg) {
  rows((const job_t*)arg);
  return NULL;
}

int orc_simd_available(void) {
  __builtin_cpu_init();
  return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

int orc_matvec_simd_mt(int type, const uint8_t* w, const float* x, float* y, size_t m, size_t k,
                       int threads) {
  if (type != ORC_Q4_0 && type != ORC_Q4_1 && type != ORC_Q8_0) return ORC_ERR_UNSUPPORTED_TYPE;
  if (k == 0 || k % 32 != 0) return ORC_ERR_INVALID_SHAPE;
  if (!orc_simd_available()) return ORC_ERR_UNSUPPORTED_TYPE;
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  job_t jobs[256];
  pthread_t tid[256];
  const size_t per = (m + (size_t)threads - 1) / (size_t)threads;
  int started = 0;
  for (int t = 0; t < threads; t++) {
    const size_t r0 = (size_t)t * per, r1 = r0 + per < m ? r0 + per : m;
    if (r0 >= r1) break;
    jobs[t] = (job_t){type, w, x, y, r0, r1, k};
    if (t == 0) continue; /* the calling thread takes range 0 */
    if (pthread_create(&tid[t], NULL, worker, &jobs[t]) != 0) {
      rows(&jobs[t]); /* no thread: run the range here */
      tid[t] = 0;
    }
    started = t + 1;
  }
  if (m > 0) rows(&jobs[0]);
  for (int t = 1; t < started; t++)
    if (tid[t]) pthread_join(tid[t], NULL);
  return ORC_OK;
}
