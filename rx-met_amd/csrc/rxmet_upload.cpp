// rxmet_upload.cpp — asynchronous host-to-device copies of the small per-call tables.
//
// hipMemcpyAsync from pageable host memory goes through the runtime's own staging and returns
// only once the copy is done, i.e. after everything queued before it on the stream: the host
// then prepares the next call while the GPU idles.  Copies from pinned memory are queued and
// return at once.  Each device has a ring of pinned slots; a slot is reused after the copy
// that last read it has completed (its event), so a caller's table may change right after the
// call returns.
#include <cstring>
#include <mutex>

#include "rxmet_common.h"

namespace rxmet {
namespace {

constexpr int kSlots = 16;
constexpr int kMaxDevices = 64;
constexpr size_t kMinSlotBytes = 64 << 10;

struct Slot {
  void *p = nullptr;
  size_t cap = 0;
  hipEvent_t ev = nullptr;
  bool pending = false;
};

struct Ring {
  std::mutex mu;
  Slot slot[kSlots];
  int next = 0;
};

Ring g_rings[kMaxDevices];

}  // namespace

int upload(void *dst, const void *src, size_t bytes, hipStream_t stream) {
  if (bytes == 0) return 0;
  int dev = 0;
  RXMET_CHECK_HIP(hipGetDevice(&dev));
  RXMET_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "device ordinal out of range");
  Ring &r = g_rings[dev];
  std::lock_guard<std::mutex> lock(r.mu);
  Slot &s = r.slot[r.next];
  r.next = (r.next + 1) % kSlots;
  if (s.pending) {
    RXMET_CHECK_HIP(hipEventSynchronize(s.ev));
    s.pending = false;
  }
  if (s.cap < bytes) {
    if (s.p != nullptr) RXMET_CHECK_HIP(hipHostFree(s.p));
    s.p = nullptr;
    s.cap = 0;
    const size_t cap = bytes > kMinSlotBytes ? bytes : kMinSlotBytes;
    RXMET_CHECK_HIP(hipHostMalloc(&s.p, cap, hipHostMallocDefault));
    s.cap = cap;
  }
  if (s.ev == nullptr) RXMET_CHECK_HIP(hipEventCreateWithFlags(&s.ev, hipEventDisableTiming));
  std::memcpy(s.p, src, bytes);
  RXMET_CHECK_HIP(hipMemcpyAsync(dst, s.p, bytes, hipMemcpyHostToDevice, stream));
  RXMET_CHECK_HIP(hipEventRecord(s.ev, stream));
  s.pending = true;
  return 0;
}

}  // namespace rxmet
