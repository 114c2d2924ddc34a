// Per-device helper streams and their event pools (declared in pd_common.hpp).
#include <mutex>
#include <string>
#include <vector>

#include "pd_common.hpp"

namespace pd {

namespace {
constexpr int AUX_MAX_DEVICES = 64;
constexpr int AUX_MAX_EVENTS = 256;  // reserved up front, so a pool never moves
struct AuxSlot {
  hipStream_t st = nullptr;
  std::vector<hipEvent_t> ev;
  std::mutex use;  // held by one entry point's enqueue sequence at a time
};
std::mutex g_aux_mu;
AuxSlot g_aux[AUX_MAX_DEVICES][2];
}  // namespace

int aux_stream(int which, int n_events, AuxStream& out) {
  int dev = -1;
  if (which < 0 || which > 1 || n_events < 0 || n_events > AUX_MAX_EVENTS)
    return fail(PD_EINVAL, "aux_stream: bad arguments (at most 256 events)");
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= AUX_MAX_DEVICES)
    return fail(PD_ELAUNCH, "aux_stream: no current HIP device in range");
  if (out.lease.owns_lock()) return fail(PD_EINVAL, "aux_stream: this AuxStream already holds a lease");
  AuxSlot& a = g_aux[dev][which];
  // Take the slot for this call first (waiting for another thread's call to finish its
  // enqueue), then grow its stream / event pool under the creation lock.
  std::unique_lock<std::mutex> lease(a.use);
  std::lock_guard<std::mutex> lock(g_aux_mu);
  hipError_t e = hipSuccess;
  if (!a.st) {
    hipStream_t st = nullptr;
    e = hipStreamCreateWithFlags(&st, hipStreamNonBlocking);
    if (e == hipSuccess) {
      a.st = st;
      a.ev.reserve(AUX_MAX_EVENTS);
    }
  }
  while (e == hipSuccess && (int)a.ev.size() < n_events) {
    hipEvent_t ev = nullptr;
    e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e == hipSuccess) a.ev.push_back(ev);
  }
  if (e != hipSuccess) return fail(PD_ELAUNCH, std::string("aux_stream: ") + hipGetErrorString(e));
  out.st = a.st;
  out.ev = a.ev.data();
  out.lease = std::move(lease);
  return PD_OK;
}

}  // namespace pd
