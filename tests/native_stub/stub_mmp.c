/* Host-only stand-in for the libmmp_hip.so entry points the native gate
 * calls (test infrastructure: no device).  Allocations are host memory;
 * kernel entry points record their arguments (and a copy of a launch's
 * parameter block) instead of running, so a test can compare what the
 * native gate would launch with what the Python path computes. */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static int64_t g_calls[64][8];
static int g_ncalls = 0;
static unsigned char g_params[4096];
static size_t g_param_bytes = 0;
static long long g_allocs = 0, g_frees = 0;

static void rec(int64_t a, int64_t b, int64_t c, int64_t d, int64_t e, int64_t f, int64_t g,
                int64_t h) {
  if (g_ncalls >= 64) return;
  int64_t *r = g_calls[g_ncalls++];
  r[0] = a; r[1] = b; r[2] = c; r[3] = d; r[4] = e; r[5] = f; r[6] = g; r[7] = h;
}

int mmp_alloc(size_t bytes, void **p) {
  *p = aligned_alloc(256, (bytes + 255) / 256 * 256);
  ++g_allocs;
  return *p ? 0 : 3;
}
int mmp_free(void *p) { free(p); ++g_frees; return 0; }
int mmp_unary(int op, int dt, int64_t n, const void *x, void *out) {
  rec(1, op, dt, n, (int64_t)(uintptr_t)x, (int64_t)(uintptr_t)out, 0, 0);
  return 0;
}
int mmp_binary(int op, int dt, int64_t n, const void *a, const void *b, void *out) {
  rec(2, op, dt, n, (int64_t)(uintptr_t)a, (int64_t)(uintptr_t)b, (int64_t)(uintptr_t)out, 0);
  return 0;
}
int mmp_binary_scalar(int op, int dt, int64_t n, const void *a, const void *s, int side,
                      void *out) {
  int64_t bits = 0;
  memcpy(&bits, s, 8);
  rec(3, op, dt, n, (int64_t)(uintptr_t)a, bits, side, (int64_t)(uintptr_t)out);
  return 0;
}
int mmp_rtc_launch(void *k, const uint32_t *grid, const uint32_t *block, uint32_t shared,
                   void **args) {
  rec(4, (int64_t)(uintptr_t)k, grid[0], grid[1], grid[2], block[0], shared, 0);
  if (g_param_bytes && g_param_bytes <= sizeof g_params) memcpy(g_params, args[0], g_param_bytes);
  return 0;
}
int mmp_rtc_compile(const char *src, const char *name, const char *opts, void **k) {
  (void)src; (void)name; (void)opts;
  *k = (void *)(uintptr_t)0x4000;
  return 0;
}
const char *mmp_last_error(void) { return "stub"; }
int mmp_reduce(int op, int dt, int odt, int64_t outer, int64_t len, int64_t inner, const void *x,
               void *out) {
  rec(5, op, dt, odt, outer, len, inner, (int64_t)(uintptr_t)out);
  (void)x;
  return 0;
}
int mmp_argreduce(int op, int dt, int64_t outer, int64_t len, int64_t inner, const void *x,
                  int64_t *out) {
  rec(6, op, dt, outer, len, inner, (int64_t)(uintptr_t)x, (int64_t)(uintptr_t)out);
  for (int64_t i = 0; i < outer * inner; ++i) out[i] = 7;  /* a recognisable index */
  return 0;
}
int mmp_h2d(void *dst, const void *src, size_t n) { memcpy(dst, src, n); return 0; }
int mmp_d2h(void *dst, const void *src, size_t n) { memcpy(dst, src, n); return 0; }

/* test accessors */
void stub_reset(size_t param_bytes) { g_ncalls = 0; g_param_bytes = param_bytes; }
int stub_ncalls(void) { return g_ncalls; }
int64_t stub_call(int i, int j) { return g_calls[i][j]; }
const unsigned char *stub_params(void) { return g_params; }
long long stub_live(void) { return g_allocs - g_frees; }
