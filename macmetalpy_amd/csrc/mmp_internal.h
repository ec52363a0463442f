// mmp_internal.h -- shared host-side helpers of libmmp_hip.so (not ABI).
#pragma once
#include <mutex>

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mmp_hip.h"

namespace mmpi {

// Library stream (created by mmp_init).  All kernels and copies go here.
hipStream_t stream();
// Ensure mmp_init ran (lazily initialising device 0); returns status.
int ensure_init();
// Number of compute units of the current device.
int cu_count();
// Whether mmp_init has run, and the library's device.
bool initialized();
int device_id();
// Resolve and clear the device's copy of mmp_reduce_noalloc's static
// scratch (reduce.hip); called once per device by mmp_init.
int noalloc_setup(int device);

// Record an error message for mmp_last_error and return `code`.
int fail(int code, const char *fmt, ...);
// Check a HIP status; on error record it and return MMP_E_HIP.
int check_hip(hipError_t e, const char *what);
// Check the last launch; returns 0 or MMP_E_HIP (also honours injection).
int check_launch(const char *what);
// Fault-injection counters (mmp_debug_fail_next).
bool inject(int kind);

// Per-device scratch memory owned by the library (grown on demand, never
// shrunk).  Used for reduction partials, completion tickets and scan tile
// descriptors.  The memory is zero-filled when first allocated; kernels
// that use counters leave them at zero when they finish.
void *scratch(int slot, size_t bytes, int *status);
enum { SCRATCH_REDUCE_PARTIALS = 0, SCRATCH_REDUCE_TICKETS = 1,
       SCRATCH_SCAN_FLAGS = 2, SCRATCH_SCAN_VALUES = 3,
       SCRATCH_SCAN_COUNTER = 4, SCRATCH_NSLOTS = 5 };
// Monotone call counter used to tag scan tile flags with a generation, so
// the flag array never needs clearing between calls (atomic: concurrent
// callers never share a generation).
uint32_t next_generation();

// Held by every entry point that uses the shared scratch slots, from the
// slot lookup through the kernel launches: a concurrent call on another
// host thread could otherwise grow (free and replace) a slot between this
// call's lookup and its launch.  Launches of all callers go to the one
// library stream, so the kernels themselves run in enqueue order.
std::mutex &launch_mutex();

// Flags of device-side bounded waits that ran out, in pinned host memory
// that kernels write with system-scope stores: word 0 scan look-back,
// word 1 reduction combine.  Read (and cleared) by the host after a stream
// synchronisation, so checking them costs no device round trip.
unsigned *wait_flags();
// Flags raised since the last call (bit 0 scan row tail, bit 1 reduction),
// cleared.
// Only meaningful after the stream has been synchronised.
uint32_t take_wait_flags();

// Parameters of the next bounded cross-workgroup wait.  Normally the spin
// limit is large and readers expect the call's own tag (tag_offset 0).
// mmp_debug_fail_next(4, n) makes the n-th next split reduction or scan
// wait for a tag its writers never write, with a spin limit of 64: a split
// reduction's wait runs out at once and the kernel still finishes (a test
// of the timeout reporting that needs no hung or faulting kernel); a scan
// finds no predecessor's descriptor, so every tile sums its predecessors'
// inputs itself (a test of that path: the result stays exact).
struct WaitParams {
  long long spin_limit;
  unsigned tag_offset;
};
WaitParams wait_params();

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace mmpi

// Dispatch a dtype code onto a C++ type.  BODY is a lambda-like block that
// uses the type alias `T`.
#define MMP_DISPATCH_ALL(dtype, ...)                                          \
  switch (dtype) {                                                            \
    case MMP_BOOL: { typedef bool T; __VA_ARGS__ }                            \
    case MMP_I16: { typedef mmp_i16 T; __VA_ARGS__ }                          \
    case MMP_U16: { typedef mmp_u16 T; __VA_ARGS__ }                          \
    case MMP_I32: { typedef mmp_i32 T; __VA_ARGS__ }                          \
    case MMP_U32: { typedef mmp_u32 T; __VA_ARGS__ }                          \
    case MMP_I64: { typedef mmp_i64 T; __VA_ARGS__ }                          \
    case MMP_U64: { typedef mmp_u64 T; __VA_ARGS__ }                          \
    case MMP_F16: { typedef mmp_half T; __VA_ARGS__ }                         \
    case MMP_F32: { typedef float T; __VA_ARGS__ }                            \
    case MMP_F64: { typedef double T; __VA_ARGS__ }                           \
    default:                                                                  \
      return mmpi::fail(MMP_E_UNSUPPORTED, "unsupported dtype code %d",       \
                        (int)(dtype));                                        \
  }
