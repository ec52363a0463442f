// stubs.hip -- entry points not implemented yet (replaced as they land).
#include "mmp_internal.h"

extern "C" int mmp_matmul(int, int64_t, int64_t, int64_t, int64_t, const void *, int64_t, int64_t,
                          const void *, int64_t, int64_t, void *, int64_t, int64_t) {
  return mmpi::fail(MMP_E_UNSUPPORTED, "mmp_matmul not implemented");
}
