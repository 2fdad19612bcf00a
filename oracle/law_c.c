/* Plain-C restatement of the W4A8 hot loops -- TEST INFRASTRUCTURE.
 *
 * A second, independent implementation of the reference's integer law,
 * used by tests/ as a cross-check of oracle/law.py and by bench.py's
 * cpu_baseline leg as the multi-threaded CPU baseline.  It reads the wire
 * image directly (ref/w4a8_ref.py:349-370 layout) as the FPGA engine does
 * (rtl/matvec_engine.sv walks one 64-byte beat per group).
 *
 *   orc_matvec_y32_img   ref/w4a8_ref.py:254-289 over a row image
 *   orc_dynq8            ref/fixedpoint.py:24-33
 *   orc_argmax           gen_layer_script.py:1424-1433 (first max wins)
 *
 * Build: make -C oracle   (gcc -O3 -fopenmp, no other dependency)
 */
#include <stdint.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_OK 0
#define ORC_E_SHAPE (-1)
#define ORC_E_Y32_OVF (-4)

static int64_t rshr64(int64_t v, int s) {
  if (s == 0) return v;
  if (s < 0) return (int64_t)((uint64_t)v << (-s));
  int64_t half = (int64_t)1 << (s - 1);
  return v >= 0 ? (v + half) >> s : -((-v + half) >> s);
}

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* y32[r] for every row of an image of nrows rows of K weights. */
int orc_matvec_y32_img(const uint8_t *img, int64_t nrows, int32_t K,
                       int32_t sh, const int8_t *x8, int32_t *y32,
                       int32_t nthreads) {
  if (K <= 0 || K % 128) return ORC_E_SHAPE;
  const int ng = K / 128;
  const int64_t stride = (int64_t)(ng + (ng + 31) / 32) * 64;
  int bad = 0;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static) reduction(| : bad)
#endif
  for (int64_t r = 0; r < nrows; ++r) {
    const uint8_t *row = img + r * stride;
    const uint8_t *sc = row + (int64_t)K / 2;
    int64_t p = 0;
    for (int g = 0; g < ng; ++g) {
      const uint8_t *wb = row + 64 * g;
      const int8_t *xg = x8 + 128 * g;
      int32_t acc = 0;
      for (int j = 0; j < 64; ++j) {
        int lo = (int)(int8_t)(uint8_t)(wb[j] << 4) >> 4;
        int hi = (int)(int8_t)wb[j] >> 4;
        acc += lo * xg[2 * j] + hi * xg[2 * j + 1];
      }
      uint32_t m = (uint32_t)sc[2 * g] | ((uint32_t)sc[2 * g + 1] << 8);
      p += (int64_t)m * acc;
    }
    int64_t y = rshr64(p, sh);
    if (y > 2147483647LL || y < -2147483647LL) bad = 1;
    y32[r] = (int32_t)y;
  }
  return bad ? ORC_E_Y32_OVF : ORC_OK;
}

int orc_dynq8(const int16_t *x16, int32_t n, int8_t *x8, int32_t *e_out) {
  int32_t mx = 0;
  for (int32_t i = 0; i < n; ++i) {
    int32_t a = x16[i] < 0 ? -(int32_t)x16[i] : x16[i];
    if (a > mx) mx = a;
  }
  int e = 0;
  while (((mx + ((1 << e) >> 1)) >> e) > 127) ++e;
  for (int32_t i = 0; i < n; ++i) {
    int64_t q = rshr64(x16[i], e);
    x8[i] = (int8_t)(q > 127 ? 127 : (q < -127 ? -127 : q));
  }
  *e_out = e;
  return ORC_OK;
}

void orc_argmax(const int32_t *y, int64_t n, int64_t *idx, int32_t *val) {
  int64_t bi = 0;
  int32_t bv = n ? y[0] : 0;
  for (int64_t i = 1; i < n; ++i)
    if (y[i] > bv) { bv = y[i]; bi = i; }
  *idx = bi;
  *val = bv;
}
