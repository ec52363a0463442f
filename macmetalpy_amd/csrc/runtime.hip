// runtime.hip -- device, stream, caching allocator, copies, events, error
// reporting, scratch memory and runtime compilation for libmmp_hip.so.
//
// Replaces MetalBackend (src/macmetalpy/_metal_backend.py:179-372) and its
// _BufferPool (:23-77).  Differences by design:
//  * one in-order HIP stream per process (default priority); the caching
//    pool's frees are stream-ordered, so a freed block can be handed to the
//    next allocation immediately -- the reference defers reuse until a
//    synchronize() (_metal_backend.py:155-162) because Metal command buffers
//    are not ordered against host reuse;
//  * every call reports failures through a status code + thread-local
//    message instead of the metalgpu ABI's silent `void`;
//  * kernels are precompiled gfx950 code objects; only fused expressions and
//    user RawKernels go through hiprtc, cached by source text.
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <hip/hiprtc.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "mmp_internal.h"

#include <atomic>
#include <chrono>

namespace {

struct Device {
  bool ready = false;
  int id = -1;
  hipStream_t stream = nullptr;
  int cus = 0;
  int wave = 64;
  int max_threads = 1024;
  int64_t total_mem = 0;
  std::string arch;
};

Device g_dev;
std::mutex g_mu;                 // guards g_dev init, pool, rtc cache
thread_local std::string g_err;  // mmp_last_error

// ---- caching pool --------------------------------------------------------
// Sizes are rounded to 4 KiB below 2 MiB and to 2 MiB above; a free block
// is reused for a request of the same rounded size (or up to 25% larger
// for big blocks).  Minimum 4 KiB so tiny arrays never share a page with
// another allocation.
std::multimap<size_t, void *> g_free;         // rounded size -> block
std::unordered_map<void *, size_t> g_live;    // block -> rounded size
size_t g_in_use = 0, g_cached = 0;

size_t round_size(size_t b) {
  const size_t small = 4096, big = 2u << 20;
  if (b < big) return (b + small - 1) / small * small;
  return (b + big - 1) / big * big;
}

// ---- scratch -------------------------------------------------------------
void *g_scratch[mmpi::SCRATCH_NSLOTS] = {};
size_t g_scratch_size[mmpi::SCRATCH_NSLOTS] = {};
std::atomic<uint32_t> g_generation{0};
std::mutex g_launch_mu;
unsigned *g_wait_flags = nullptr;  // pinned host words written by kernels

// ---- fault injection (mmp_debug_fail_next) -------------------------------
int g_fail_kind = 0, g_fail_count = 0;

// ---- rtc cache -----------------------------------------------------------
struct RtcEntry {
  hipModule_t module;
  hipFunction_t fn;
};
std::unordered_map<std::string, RtcEntry> g_rtc;
// Modules by (options, source): several kernels of one source share one
// compilation (the reference's execute_kernel selects functions of one
// library, _metal_backend.py:341-356).
std::unordered_map<std::string, hipModule_t> g_rtc_mod;

int init_locked(int device) {
  if (g_dev.ready) {
    if (device == g_dev.id) return MMP_OK;
    return mmpi::fail(MMP_E_ARG, "already initialised on device %d", g_dev.id);
  }
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count <= 0)
    return mmpi::fail(MMP_E_NODEVICE, "no HIP device available (%s)",
                      e == hipSuccess ? "0 devices" : hipGetErrorString(e));
  if (device < 0 || device >= count)
    return mmpi::fail(MMP_E_ARG, "device %d out of range (%d devices)", device, count);
  if (int st = mmpi::check_hip(hipSetDevice(device), "hipSetDevice")) return st;
  hipDeviceProp_t prop;
  if (int st = mmpi::check_hip(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties"))
    return st;
  hipStream_t s;
  if (int st = mmpi::check_hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking),
                               "hipStreamCreateWithFlags"))
    return st;
  void *flags = nullptr;
  if (int st = mmpi::check_hip(hipHostMalloc(&flags, 256, hipHostMallocMapped | hipHostMallocCoherent),
                               "hipHostMalloc(wait flags)"))
    return st;
  std::memset(flags, 0, 256);
  g_wait_flags = static_cast<unsigned *>(flags);
  g_dev.stream = s;
  g_dev.id = device;
  g_dev.cus = prop.multiProcessorCount;
  g_dev.wave = prop.warpSize;
  g_dev.max_threads = prop.maxThreadsPerBlock;
  g_dev.total_mem = (int64_t)prop.totalGlobalMem;
  g_dev.arch = prop.gcnArchName;
  if (int st = mmpi::noalloc_setup(device)) return st;
  g_dev.ready = true;
  return MMP_OK;
}

void release_cached_locked() {
  for (auto &kv : g_free) {
    (void)hipFree(kv.second);
  }
  g_free.clear();
  g_cached = 0;
}

}  // namespace

// ========================================================================
// internal helpers
// ========================================================================
namespace mmpi {

int fail(int code, const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int check_hip(hipError_t e, const char *what) {
  if (e == hipSuccess) return MMP_OK;
  return fail(e == hipErrorOutOfMemory ? MMP_E_OOM : MMP_E_HIP, "%s failed: %s", what,
              hipGetErrorString(e));
}

bool inject(int kind) {
  if (g_fail_kind != kind || g_fail_count <= 0) return false;
  if (--g_fail_count == 0) {
    g_fail_kind = 0;
    return true;
  }
  return false;
}

int check_launch(const char *what) {
  if (inject(3)) return fail(MMP_E_INJECTED, "%s: injected launch failure", what);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) return MMP_OK;
  return fail(MMP_E_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
}

hipStream_t stream() { return g_dev.stream; }

int ensure_init() {
  if (g_dev.ready) return MMP_OK;
  std::lock_guard<std::mutex> lk(g_mu);
  return init_locked(0);
}

int cu_count() { return g_dev.cus; }
bool initialized() { return g_dev.ready; }
int device_id() { return g_dev.ready ? g_dev.id : -1; }

void *scratch(int slot, size_t bytes, int *status) {
  *status = MMP_OK;
  if (slot < 0 || slot >= SCRATCH_NSLOTS) {
    *status = fail(MMP_E_ARG, "bad scratch slot");
    return nullptr;
  }
  if (g_scratch_size[slot] >= bytes && g_scratch[slot]) return g_scratch[slot];
  size_t want = round_size(bytes < 65536 ? 65536 : bytes);
  // growing: wait for users of the old block before replacing it
  if (g_scratch[slot]) {
    if ((*status = check_hip(hipStreamSynchronize(g_dev.stream), "hipStreamSynchronize")))
      return nullptr;
    (void)hipFree(g_scratch[slot]);
    g_scratch[slot] = nullptr;
    g_scratch_size[slot] = 0;
  }
  void *p = nullptr;
  if ((*status = check_hip(hipMalloc(&p, want), "hipMalloc(scratch)"))) return nullptr;
  if ((*status = check_hip(hipMemsetAsync(p, 0, want, g_dev.stream), "hipMemsetAsync(scratch)"))) {
    (void)hipFree(p);
    return nullptr;
  }
  g_scratch[slot] = p;
  g_scratch_size[slot] = want;
  return p;
}

unsigned *wait_flags() { return g_wait_flags; }

uint32_t take_wait_flags() {
  if (!g_wait_flags) return 0;
  volatile unsigned *w = g_wait_flags;
  const uint32_t f = (w[0] ? 1u : 0u) | (w[1] ? 2u : 0u);
  if (f) {
    w[0] = 0;
    w[1] = 0;
  }
  return f;
}

WaitParams wait_params() {
  if (inject(4)) return WaitParams{64, 1u};
  return WaitParams{1ll << 26, 0u};
}

uint32_t next_generation() {
  // 30 usable bits (flags keep 2 state bits); 0 is never used so that
  // zero-filled scratch never matches a live generation.
  uint32_t g;
  do {
    g = (g_generation.fetch_add(1, std::memory_order_relaxed) + 1) & 0x3fffffffu;
  } while (g == 0);
  return g;
}

std::mutex &launch_mutex() { return g_launch_mu; }

}  // namespace mmpi

namespace {
// After a stream synchronisation: report device-side waits that ran out.
int check_waits() {
  const uint32_t f = mmpi::take_wait_flags();
  if (!f) return MMP_OK;
  return mmpi::fail(MMP_E_WAIT,
                    "a device-side bounded wait ran out (%s%s): a %s result computed since the "
                    "last synchronisation may be wrong",
                    (f & 1u) ? "scan row tail prefix" : "", f == 3u ? ", reduction combine" : (f == 2u ? "reduction combine" : ""),
                    f == 1u ? "cumsum / cumprod" : (f == 2u ? "reduction" : "scan or reduction"));
}
}  // namespace

// ========================================================================
// C ABI
// ========================================================================
extern "C" {

const char *mmp_last_error(void) { return g_err.c_str(); }

int mmp_init(int device) {
  std::lock_guard<std::mutex> lk(g_mu);
  return init_locked(device);
}

int mmp_device_count(int *count) {
  if (!count) return mmpi::fail(MMP_E_ARG, "null count");
  int c = 0;
  if (hipGetDeviceCount(&c) != hipSuccess) c = 0;
  *count = c;
  return MMP_OK;
}

int mmp_device_info(char *arch, int arch_len, int *cu_count, int64_t *total_mem,
                    int *wave_size, int *max_threads) {
  if (int st = mmpi::ensure_init()) return st;
  if (arch && arch_len > 0) {
    std::snprintf(arch, (size_t)arch_len, "%s", g_dev.arch.c_str());
  }
  if (cu_count) *cu_count = g_dev.cus;
  if (total_mem) *total_mem = g_dev.total_mem;
  if (wave_size) *wave_size = g_dev.wave;
  if (max_threads) *max_threads = g_dev.max_threads;
  return MMP_OK;
}

int mmp_alloc(size_t bytes, void **ptr) {
  if (!ptr) return mmpi::fail(MMP_E_ARG, "null ptr");
  *ptr = nullptr;
  if (int st = mmpi::ensure_init()) return st;
  if (mmpi::inject(1)) return mmpi::fail(MMP_E_INJECTED, "mmp_alloc: injected failure");
  const size_t want = round_size(bytes ? bytes : 1);
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_free.lower_bound(want);
  const size_t limit = want < (64u << 20) ? want : want + want / 4;
  if (it != g_free.end() && it->first <= limit) {
    void *p = it->second;
    const size_t sz = it->first;
    g_free.erase(it);
    g_cached -= sz;
    g_live[p] = sz;
    g_in_use += sz;
    *ptr = p;
    return MMP_OK;
  }
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, want);
  if (e != hipSuccess) {
    // give the cache back to the driver and retry once
    (void)hipGetLastError();
    (void)hipStreamSynchronize(g_dev.stream);
    release_cached_locked();
    e = hipMalloc(&p, want);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return mmpi::fail(MMP_E_OOM, "mmp_alloc(%zu bytes): %s", bytes, hipGetErrorString(e));
    }
  }
  g_live[p] = want;
  g_in_use += want;
  *ptr = p;
  return MMP_OK;
}

int mmp_free(void *ptr) {
  if (!ptr) return MMP_OK;
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_live.find(ptr);
  if (it == g_live.end()) return mmpi::fail(MMP_E_ARG, "mmp_free: unknown pointer %p", ptr);
  const size_t sz = it->second;
  g_live.erase(it);
  g_in_use -= sz;
  g_free.emplace(sz, ptr);
  g_cached += sz;
  return MMP_OK;
}

int mmp_empty_cache(void) {
  if (!g_dev.ready) return MMP_OK;
  std::lock_guard<std::mutex> lk(g_mu);
  if (int st = mmpi::check_hip(hipStreamSynchronize(g_dev.stream), "hipStreamSynchronize"))
    return st;
  release_cached_locked();
  return MMP_OK;
}

int mmp_memory_stats(size_t *in_use, size_t *cached) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (in_use) *in_use = g_in_use;
  if (cached) *cached = g_cached;
  return MMP_OK;
}

// ---------------------------------------------------- upload staging
// Host->device copies of up to kStageSeg bytes go through a page-locked
// ring of kStageSegs segments: the bytes are copied into the ring on the
// host and the DMA is queued on the stream without a host wait (a copy from
// pageable memory makes the runtime stage it and block).  The ring leaves a
// segment by recording an event on the stream; it re-enters that segment
// only after the event has completed, so a staged source stays intact until
// the device has read it.  Later work on the stream sees the copied bytes
// (in-order stream).  For small host arrays this turns each upload from a
// blocking round trip into a host memcpy plus a queued copy.
namespace {
// Small copies between device memory and the mapped, coherent staging
// memory below run as a kernel on the library stream instead of a DMA
// transfer.  Measured on MI355X:
//  * device -> host, copy plus stream wait: 4-24 KiB 13.0-14.3 us by kernel
//    against 19-27 us by DMA; from 32 KiB on the DMA is faster (32 KiB 11.0
//    against 14.5 us, 1 MiB 27.7 against 62.1 us: a kernel's writes to host
//    memory reach ~15 GB/s), so downloads take the kernel below 32 KiB;
//    into pageable memory (which the runtime stages) a DMA stays slow up
//    to 47 KiB (32 KiB 23.3 us, 48 KiB 11.7), so pageable destinations
//    take the kernel below 48 KiB;
//  * host -> device: the upload is followed by kernels on the same stream,
//    and there a DMA costs its hand-over to the compute queue (a 64K-element
//    float32 a + b of host arrays, two 256 KiB uploads: 66 us per call with
//    DMA uploads, 55 with kernel copies), so uploads take the kernel up to
//    the 1 MiB staging segment.
constexpr size_t kDownloadKernelBelow = 32 << 10;
constexpr size_t kDownloadPageableBelow = 48 << 10;
constexpr size_t kUploadKernelMax = 1 << 20;

__global__ __launch_bounds__(256) void k_copy_small(unsigned char *__restrict__ dst,
                                                    const unsigned char *__restrict__ src,
                                                    size_t n) {
  const size_t i0 = (size_t)blockIdx.x * 256 + threadIdx.x, step = (size_t)gridDim.x * 256;
  size_t head = 0;
  if ((((uintptr_t)dst | (uintptr_t)src) & 15) == 0) {
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    const size_t nv = n / 16;
    for (size_t i = i0; i < nv; i += step)
      reinterpret_cast<u4 *>(dst)[i] = reinterpret_cast<const u4 *>(src)[i];
    head = nv * 16;
  }
  for (size_t i = head + i0; i < n; i += step) dst[i] = src[i];
}

// The copy kernels address device memory directly; a pointer the runtime
// does not know as device memory (host memory handed to mmp_h2d / mmp_d2h,
// which DMA copies accept) takes the DMA path instead.
bool is_device_memory(const void *p) {
  hipPointerAttribute_t a;
  if (hipPointerGetAttributes(&a, p) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return a.type == hipMemoryTypeDevice;
}

// Page-locked host memory the runtime knows (hipHostMalloc'd); pageable
// memory is not.
bool is_page_locked(const void *p) {
  hipPointerAttribute_t a;
  if (hipPointerGetAttributes(&a, p) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return a.type == hipMemoryTypeHost;
}

int launch_copy_small(void *dst, const void *src, size_t n) {
  const size_t blocks = std::min<size_t>(256, (n + 16 * 256 - 1) / (16 * 256));
  hipLaunchKernelGGL(k_copy_small, dim3((unsigned)blocks), dim3(256), 0, g_dev.stream,
                     static_cast<unsigned char *>(dst), static_cast<const unsigned char *>(src), n);
  return mmpi::check_hip(hipGetLastError(), "small copy launch");
}

// Download copy: one workgroup copies the bytes into the mapped block, then
// publishes `seq` in the block's completion word with a system-scope
// release once every lane's stores are ordered before it (each lane's
// system fence, then the barrier).  The host waits for that word instead of
// the end-of-kernel signal.
__global__ __launch_bounds__(256) void k_copy_back(unsigned char *__restrict__ dst,
                                                   const unsigned char *__restrict__ src, size_t n,
                                                   unsigned *done, unsigned seq) {
  const unsigned t = threadIdx.x;
  size_t head = 0;
  if ((((uintptr_t)dst | (uintptr_t)src) & 15) == 0) {
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    const size_t nv = n / 16;
    for (size_t i = t; i < nv; i += 256)
      reinterpret_cast<u4 *>(dst)[i] = reinterpret_cast<const u4 *>(src)[i];
    head = nv * 16;
  }
  for (size_t i = head + t; i < n; i += 256) dst[i] = src[i];
  __threadfence_system();
  __syncthreads();
  if (t == 0) __hip_atomic_store(done, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

constexpr size_t kStageSeg = 1 << 20;
constexpr int kStageSegs = 8;
constexpr size_t kStageAlign = 256;
std::mutex g_stage_mu;
char *g_stage = nullptr;      // kStageSegs * kStageSeg page-locked bytes
char *g_stage_dev = nullptr;  // the same bytes as the device addresses them
hipEvent_t g_stage_ev[kStageSegs] = {};
bool g_stage_pending[kStageSegs] = {};
int g_stage_seg = 0;
size_t g_stage_head = 0;  // bytes used in the current segment
bool g_stage_off = false;  // set up failed: every copy takes the blocking path

constexpr int kNotStaged = -1;

// kNotStaged: the caller copies directly; else an mmp status.
int stage_upload(void *dst, const void *src, size_t bytes) {
  std::lock_guard<std::mutex> lk(g_stage_mu);
  if (g_stage_off) return kNotStaged;
  if (!g_stage) {
    void *p = nullptr;
    if (hipHostMalloc(&p, kStageSeg * kStageSegs, hipHostMallocMapped | hipHostMallocCoherent) !=
            hipSuccess ||
        !p) {
      (void)hipGetLastError();
      g_stage_off = true;
      return kNotStaged;
    }
    for (int i = 0; i < kStageSegs; ++i) {
      if (hipEventCreateWithFlags(&g_stage_ev[i], hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        for (int j = 0; j < i; ++j) (void)hipEventDestroy(g_stage_ev[j]);
        (void)hipHostFree(p);
        g_stage_off = true;
        return kNotStaged;
      }
    }
    void *dp = nullptr;
    if (hipHostGetDevicePointer(&dp, p, 0) != hipSuccess || !dp) {
      (void)hipGetLastError();
      for (int j = 0; j < kStageSegs; ++j) (void)hipEventDestroy(g_stage_ev[j]);
      (void)hipHostFree(p);
      g_stage_off = true;
      return kNotStaged;
    }
    g_stage = static_cast<char *>(p);
    g_stage_dev = static_cast<char *>(dp);
  }
  const size_t span = (bytes + kStageAlign - 1) / kStageAlign * kStageAlign;
  if (g_stage_head + span > kStageSeg) {  // leave the segment, enter the next one
    if (int st = mmpi::check_hip(hipEventRecord(g_stage_ev[g_stage_seg], g_dev.stream),
                                 "hipEventRecord(staging)"))
      return st;
    g_stage_pending[g_stage_seg] = true;
    g_stage_seg = (g_stage_seg + 1) % kStageSegs;
    g_stage_head = 0;
    if (g_stage_pending[g_stage_seg]) {
      if (int st = mmpi::check_hip(hipEventSynchronize(g_stage_ev[g_stage_seg]),
                                   "hipEventSynchronize(staging)"))
        return st;
      g_stage_pending[g_stage_seg] = false;
    }
  }
  const size_t at = (size_t)g_stage_seg * kStageSeg + g_stage_head;
  char *slot = g_stage + at;
  std::memcpy(slot, src, bytes);
  g_stage_head += span;
  if (bytes <= kUploadKernelMax) return launch_copy_small(dst, g_stage_dev + at, bytes);
  return mmpi::check_hip(hipMemcpyAsync(dst, slot, bytes, hipMemcpyHostToDevice, g_dev.stream),
                         "hipMemcpyAsync(H2D, staged)");
}

// Small device -> host copies: one workgroup writes the bytes into a
// mapped, coherent page-locked block and then a completion word behind
// them; the host polls that word (bounded: after kBackSpin it waits for
// the stream instead, then the word must be there), then copies the bytes
// out.  Stream order puts the copy after every kernel queued before it,
// and a word seen means the bytes before it are visible.
std::mutex g_back_mu;
char *g_back = nullptr, *g_back_dev = nullptr;
bool g_back_off = false;
unsigned g_back_seq = 0;
constexpr size_t kBackWord = kDownloadPageableBelow;  // offset of the completion word
constexpr auto kBackSpin = std::chrono::microseconds(200);

int small_download(void *dst, const void *src, size_t bytes) {
  std::lock_guard<std::mutex> lk(g_back_mu);
  if (g_back_off) return kNotStaged;
  if (!g_back) {
    void *p = nullptr;
    if (hipHostMalloc(&p, kBackWord + 256, hipHostMallocMapped | hipHostMallocCoherent) !=
            hipSuccess ||
        !p) {
      (void)hipGetLastError();
      g_back_off = true;
      return kNotStaged;
    }
    void *dp = nullptr;
    if (hipHostGetDevicePointer(&dp, p, 0) != hipSuccess || !dp) {
      (void)hipGetLastError();
      (void)hipHostFree(p);
      g_back_off = true;
      return kNotStaged;
    }
    g_back = static_cast<char *>(p);
    g_back_dev = static_cast<char *>(dp);
    __atomic_store_n(reinterpret_cast<unsigned *>(g_back + kBackWord), 0u, __ATOMIC_RELAXED);
  }
  if (++g_back_seq == 0) g_back_seq = 1;  // 0 is the word's initial value
  const unsigned seq = g_back_seq;
  hipLaunchKernelGGL(k_copy_back, dim3(1), dim3(256), 0, g_dev.stream,
                     reinterpret_cast<unsigned char *>(g_back_dev),
                     static_cast<const unsigned char *>(src), bytes,
                     reinterpret_cast<unsigned *>(g_back_dev + kBackWord), seq);
  if (int st = mmpi::check_hip(hipGetLastError(), "download copy launch")) return st;
  // acquire loads: the bytes read below are ordered after the word
  unsigned *done = reinterpret_cast<unsigned *>(g_back + kBackWord);
  const auto t0 = std::chrono::steady_clock::now();
  bool seen = false;
  for (unsigned i = 1;; ++i) {
    if (__atomic_load_n(done, __ATOMIC_ACQUIRE) == seq) {
      seen = true;
      break;
    }
    if ((i & 63) == 0 && std::chrono::steady_clock::now() - t0 > kBackSpin) break;
  }
  if (!seen) {
    if (int st = mmpi::check_hip(hipStreamSynchronize(g_dev.stream), "hipStreamSynchronize"))
      return st;
    if (__atomic_load_n(done, __ATOMIC_ACQUIRE) != seq)
      return mmpi::fail(MMP_E_HIP, "small download: completion word not written");
  }
  std::memcpy(dst, g_back, bytes);
  return MMP_OK;
}
}  // namespace

int mmp_h2d(void *dst, const void *src, size_t bytes) {
  if (int st = mmpi::ensure_init()) return st;
  if (bytes == 0) return MMP_OK;
  if (!dst || !src) return mmpi::fail(MMP_E_ARG, "null pointer");
  if (bytes <= kStageSeg && is_device_memory(dst)) {
    const int st = stage_upload(dst, src, bytes);
    if (st != kNotStaged) return st;
  }
  if (int st = mmpi::check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_dev.stream),
                               "hipMemcpyAsync(H2D)"))
    return st;
  return mmpi::check_hip(hipStreamSynchronize(g_dev.stream), "hipStreamSynchronize");
}

int mmp_d2h(void *dst, const void *src, size_t bytes) {
  if (int st = mmpi::ensure_init()) return st;
  if (bytes == 0) return MMP_OK;
  if (!dst || !src) return mmpi::fail(MMP_E_ARG, "null pointer");
  if (bytes < kDownloadPageableBelow && is_device_memory(src) &&
      (bytes < kDownloadKernelBelow || !is_page_locked(dst))) {
    const int st = small_download(dst, src, bytes);
    if (st == MMP_OK) return check_waits();
    if (st != kNotStaged) return st;
  }
  if (int st = mmpi::check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_dev.stream),
                               "hipMemcpyAsync(D2H)"))
    return st;
  if (int st = mmpi::check_hip(hipStreamSynchronize(g_dev.stream), "hipStreamSynchronize"))
    return st;
  return check_waits();
}

// ---------------------------------------------------- pinned host blocks
// Page-locked host memory for results copied back to the host: a DMA into
// it runs at the link rate, where a copy into pageable memory is staged by
// the runtime.  Blocks are cached by their rounded size (hipHostMalloc is
// expensive); at most kHostCacheMax bytes stay cached, and at most
// kHostLiveMax bytes may be handed out at once (callers fall back to
// pageable memory beyond that).
namespace {
constexpr size_t kHostRound = 64 << 10;
constexpr size_t kHostCacheMax = 2ull << 30;
constexpr size_t kHostLiveMax = 4ull << 30;
std::multimap<size_t, void *> g_host_free;          // rounded size -> block
std::unordered_map<void *, size_t> g_host_live;     // block -> rounded size
size_t g_host_cached = 0, g_host_out = 0;
}  // namespace

int mmp_host_alloc(size_t bytes, void **ptr) {
  if (int st = mmpi::ensure_init()) return st;
  if (!ptr) return mmpi::fail(MMP_E_ARG, "null pointer");
  *ptr = nullptr;
  const size_t r = ((bytes ? bytes : 1) + kHostRound - 1) / kHostRound * kHostRound;
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_host_out + r > kHostLiveMax)
    return mmpi::fail(MMP_E_OOM, "pinned host blocks in use exceed %zu bytes", kHostLiveMax);
  void *p = nullptr;
  auto it = g_host_free.find(r);
  if (it != g_host_free.end()) {
    p = it->second;
    g_host_free.erase(it);
    g_host_cached -= r;
  } else if (hipHostMalloc(&p, r, hipHostMallocDefault) != hipSuccess || !p) {
    (void)hipGetLastError();
    return mmpi::fail(MMP_E_OOM, "hipHostMalloc(%zu) failed", r);
  }
  g_host_live[p] = r;
  g_host_out += r;
  *ptr = p;
  return MMP_OK;
}

int mmp_host_free(void *ptr) {
  if (!ptr) return MMP_OK;
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_host_live.find(ptr);
  if (it == g_host_live.end()) return mmpi::fail(MMP_E_ARG, "not a pinned host block");
  const size_t r = it->second;
  g_host_live.erase(it);
  g_host_out -= r;
  if (g_host_cached + r <= kHostCacheMax) {
    // Insert ahead of the blocks of the same size, so find() hands back the
    // most recently released (still mapped in the TLB) block first.
    g_host_free.emplace_hint(g_host_free.lower_bound(r), r, ptr);
    g_host_cached += r;
    return MMP_OK;
  }
  return mmpi::check_hip(hipHostFree(ptr), "hipHostFree");
}

int mmp_d2d(void *dst, const void *src, size_t bytes) {
  if (int st = mmpi::ensure_init()) return st;
  if (bytes == 0) return MMP_OK;
  if (!dst || !src) return mmpi::fail(MMP_E_ARG, "null pointer");
  return mmpi::check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_dev.stream),
                         "hipMemcpyAsync(D2D)");
}

int mmp_sync(void) {
  if (!g_dev.ready) return MMP_OK;
  if (int st = mmpi::check_hip(hipStreamSynchronize(g_dev.stream), "hipStreamSynchronize"))
    return st;
  return check_waits();
}

int mmp_stream(void **stream) {
  if (!stream) return mmpi::fail(MMP_E_ARG, "null stream pointer");
  *stream = g_dev.ready ? static_cast<void *>(g_dev.stream) : nullptr;
  return MMP_OK;
}

int mmp_event_create(void **ev) {
  if (int st = mmpi::ensure_init()) return st;
  if (!ev) return mmpi::fail(MMP_E_ARG, "null event");
  hipEvent_t e;
  if (int st = mmpi::check_hip(hipEventCreate(&e), "hipEventCreate")) return st;
  *ev = (void *)e;
  return MMP_OK;
}

int mmp_event_record(void *ev) {
  if (int st = mmpi::ensure_init()) return st;
  return mmpi::check_hip(hipEventRecord((hipEvent_t)ev, g_dev.stream), "hipEventRecord");
}

int mmp_event_elapsed_ms(void *start, void *end, float *ms) {
  if (int st = mmpi::check_hip(hipEventSynchronize((hipEvent_t)end), "hipEventSynchronize"))
    return st;
  return mmpi::check_hip(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end),
                         "hipEventElapsedTime");
}

int mmp_event_destroy(void *ev) {
  return mmpi::check_hip(hipEventDestroy((hipEvent_t)ev), "hipEventDestroy");
}

// ---- runtime compilation -------------------------------------------------
// Compile `src`; when `name_expr` is given (e.g. "&kernel" for a kernel
// without extern "C"), also return its lowered (mangled) symbol name.
static int rtc_compile_code(const char *src, const char *options, const char *arch,
                            std::vector<char> *code, const char *name_expr = nullptr,
                            std::string *lowered = nullptr) {
  hiprtcProgram prog;
  hiprtcResult r = hiprtcCreateProgram(&prog, src, "mmp_rtc.hip", 0, nullptr, nullptr);
  if (r != HIPRTC_SUCCESS)
    return mmpi::fail(MMP_E_RTC, "hiprtcCreateProgram: %s", hiprtcGetErrorString(r));
  if (name_expr) hiprtcAddNameExpression(prog, name_expr);
  // split options on whitespace
  std::vector<std::string> opts;
  std::string a = std::string("--offload-arch=") + arch;
  opts.push_back(a);
  if (options) {
    std::string cur;
    for (const char *p = options;; ++p) {
      if (*p == 0 || *p == ' ' || *p == '\t' || *p == '\n') {
        if (!cur.empty()) opts.push_back(cur);
        cur.clear();
        if (*p == 0) break;
      } else {
        cur.push_back(*p);
      }
    }
  }
  std::vector<const char *> argv;
  for (auto &s : opts) argv.push_back(s.c_str());
  r = hiprtcCompileProgram(prog, (int)argv.size(), argv.data());
  if (r != HIPRTC_SUCCESS) {
    size_t lsz = 0;
    hiprtcGetProgramLogSize(prog, &lsz);
    std::string log(lsz + 1, '\0');
    if (lsz) hiprtcGetProgramLog(prog, &log[0]);
    hiprtcDestroyProgram(&prog);
    if (log.size() > 900) log.resize(900);
    return mmpi::fail(MMP_E_RTC, "hiprtc compile failed: %s", log.c_str());
  }
  size_t csz = 0;
  hiprtcGetCodeSize(prog, &csz);
  code->resize(csz);
  hiprtcGetCode(prog, code->data());
  if (name_expr && lowered) {
    const char *ln = nullptr;
    if (hiprtcGetLoweredName(prog, name_expr, &ln) == HIPRTC_SUCCESS && ln) *lowered = ln;
  }
  hiprtcDestroyProgram(&prog);
  return MMP_OK;
}

int mmp_rtc_build(const char *src, const char *options, const char *arch, void *code,
                  size_t code_cap, size_t *code_size) {
  if (!src) return mmpi::fail(MMP_E_ARG, "null source");
  std::vector<char> buf;
  if (int st = rtc_compile_code(src, options, arch ? arch : "gfx950", &buf)) return st;
  if (code_size) *code_size = buf.size();
  if (code && code_cap >= buf.size()) std::memcpy(code, buf.data(), buf.size());
  return MMP_OK;
}

int mmp_rtc_compile(const char *src, const char *name, const char *options, void **kernel) {
  if (!src || !name || !kernel) return mmpi::fail(MMP_E_ARG, "null argument");
  if (int st = mmpi::ensure_init()) return st;
  if (mmpi::inject(2)) return mmpi::fail(MMP_E_INJECTED, "mmp_rtc_compile: injected failure");
  std::string key = std::string(name) + '\x01' + (options ? options : "") + '\x01' + src;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_rtc.find(key);
    if (it != g_rtc.end()) {
      *kernel = (void *)it->second.fn;
      return MMP_OK;
    }
  }
  std::string arch = g_dev.arch;
  const size_t colon = arch.find(':');
  if (colon != std::string::npos) arch.resize(colon);
  const std::string mkey = std::string(options ? options : "") + '\x01' + src;
  hipModule_t mod = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_rtc_mod.find(mkey);
    if (it != g_rtc_mod.end()) mod = it->second;
  }
  std::vector<char> code;
  if (!mod) {
    if (int st = rtc_compile_code(src, options, arch.c_str(), &code)) return st;
    if (int st = mmpi::check_hip(hipModuleLoadData(&mod, code.data()), "hipModuleLoadData"))
      return st;
    std::lock_guard<std::mutex> lk(g_mu);
    g_rtc_mod[mkey] = mod;
  }
  hipFunction_t fn;
  hipError_t e = hipModuleGetFunction(&fn, mod, name);
  if (e != hipSuccess) {
    // not extern "C": recompile asking hiprtc for the mangled name (the
    // shared module stays loaded for the source's other kernels)
    (void)hipGetLastError();
    std::string expr = std::string("&") + name, lowered;
    if (int st = rtc_compile_code(src, options, arch.c_str(), &code, expr.c_str(), &lowered))
      return st;
    if (lowered.empty())
      return mmpi::fail(MMP_E_RTC, "kernel '%s' not found in compiled source", name);
    if (int st = mmpi::check_hip(hipModuleLoadData(&mod, code.data()), "hipModuleLoadData"))
      return st;
    e = hipModuleGetFunction(&fn, mod, lowered.c_str());
    if (e != hipSuccess) {
      (void)hipModuleUnload(mod);
      return mmpi::fail(MMP_E_RTC, "kernel '%s' (%s) not found in compiled source (%s)", name,
                        lowered.c_str(), hipGetErrorString(e));
    }
  }
  std::lock_guard<std::mutex> lk(g_mu);
  g_rtc[key] = RtcEntry{mod, fn};
  *kernel = (void *)fn;
  return MMP_OK;
}

int mmp_rtc_launch(void *kernel, const uint32_t *grid3, const uint32_t *block3,
                   uint32_t shared_bytes, void **args) {
  if (int st = mmpi::ensure_init()) return st;
  if (!kernel || !grid3 || !block3) return mmpi::fail(MMP_E_ARG, "null argument");
  if (grid3[0] == 0 || grid3[1] == 0 || grid3[2] == 0) return MMP_OK;
  if (mmpi::inject(3)) return mmpi::fail(MMP_E_INJECTED, "mmp_rtc_launch: injected failure");
  hipError_t e = hipModuleLaunchKernel((hipFunction_t)kernel, grid3[0], grid3[1], grid3[2],
                                       block3[0], block3[1], block3[2], shared_bytes,
                                       g_dev.stream, args, nullptr);
  return mmpi::check_hip(e, "hipModuleLaunchKernel");
}

int mmp_rtc_launch_threads(void *kernel, const uint32_t *threads3, const uint32_t *block3,
                           uint32_t shared_bytes, void **args) {
  if (int st = mmpi::ensure_init()) return st;
  if (!kernel || !threads3 || !block3) return mmpi::fail(MMP_E_ARG, "null argument");
  if (threads3[0] == 0 || threads3[1] == 0 || threads3[2] == 0) return MMP_OK;
  if (block3[0] == 0 || block3[1] == 0 || block3[2] == 0 ||
      (uint64_t)block3[0] * block3[1] * block3[2] > 1024)
    return mmpi::fail(MMP_E_ARG, "mmp_rtc_launch_threads: bad workgroup %ux%ux%u", block3[0],
                      block3[1], block3[2]);
  if (mmpi::inject(3)) return mmpi::fail(MMP_E_INJECTED, "mmp_rtc_launch_threads: injected failure");
  // The dispatch packet counts work-items, so a grid that is not a multiple
  // of the workgroup gets a partial last workgroup per dimension: exactly
  // threads3 work-items run, no more.
  hipError_t e = hipExtModuleLaunchKernel((hipFunction_t)kernel, threads3[0], threads3[1],
                                          threads3[2], block3[0], block3[1], block3[2],
                                          shared_bytes, g_dev.stream, args, nullptr);
  return mmpi::check_hip(e, "hipExtModuleLaunchKernel");
}

int mmp_wait_status(uint32_t *flags) {
  if (!flags) return mmpi::fail(MMP_E_ARG, "null pointer");
  *flags = 0;
  if (int st = mmpi::ensure_init()) return st;
  if (int st = mmpi::check_hip(hipStreamSynchronize(g_dev.stream), "hipStreamSynchronize"))
    return st;
  *flags = mmpi::take_wait_flags();
  return MMP_OK;
}

int mmp_debug_fail_next(int kind, int count) {
  if (kind < 0 || kind > 4 || count < 0) return mmpi::fail(MMP_E_ARG, "bad injection request");
  g_fail_kind = count > 0 ? kind : 0;
  g_fail_count = count;
  return MMP_OK;
}

}  // extern "C"
