// SlotRing: module-scope scratch slots shared by launches on any stream of
// one device (declared in lh_internal.hpp). Host code only.
#include <atomic>
#include <mutex>

#include "lh_internal.hpp"

namespace lh {

struct SlotRing::Dev {
  std::mutex mu[kMaxSlots];
  hipEvent_t ev[kMaxSlots] = {};
  bool recorded[kMaxSlots] = {};
  std::atomic<unsigned> next{0};
};

SlotRing::Dev *SlotRing::dev(int d) {
  static std::mutex init_mu;
  std::lock_guard<std::mutex> lk(init_mu);
  if (!devs_[d]) devs_[d] = new Dev();  // lives until the process ends
  return devs_[d];
}

hipError_t SlotRing::take(hipStream_t st, Lease &lease) {
  lease.release(true);
  int d = 0;
  hipError_t e = hipGetDevice(&d);
  if (e != hipSuccess) return e;
  if (d < 0 || d >= kMaxDevices || n_ < 1 || n_ > kMaxSlots) return hipErrorInvalidValue;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  e = hipStreamIsCapturing(st, &cs);
  if (e != hipSuccess) return e;
  Dev *dv = dev(d);
  const int slot = (int)(dv->next.fetch_add(1, std::memory_order_relaxed) % (unsigned)n_);
  dv->mu[slot].lock();
  lease.ring_ = this;
  lease.dev_ = d;
  lease.slot_ = slot;
  lease.st_ = st;
  lease.capturing_ = cs != hipStreamCaptureStatusNone;
  if (!lease.capturing_ && dv->recorded[slot]) {
    e = hipStreamWaitEvent(st, dv->ev[slot], 0);
    if (e != hipSuccess) {
      lease.release(false);
      return e;
    }
  }
  return hipSuccess;
}

hipError_t SlotRing::Lease::release(bool record) {
  if (!ring_ || slot_ < 0) return hipSuccess;
  Dev *dv = ring_->devs_[dev_];
  hipError_t e = hipSuccess;
  if (record && !capturing_) {
    if (!dv->ev[slot_]) e = hipEventCreateWithFlags(&dv->ev[slot_], hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(dv->ev[slot_], st_);
    dv->recorded[slot_] = dv->recorded[slot_] || e == hipSuccess;
  }
  dv->mu[slot_].unlock();
  ring_ = nullptr;
  slot_ = -1;
  return e;
}

}  // namespace lh
