// Per-thread pinned host buffers (status mailboxes, staging of the divide-and-conquer node lists)
// and their release through mpq_release_thread_resources().
#include <vector>

#include "common.h"

namespace mpq {
namespace {

struct PinnedSlot {
  void** host;
  void** dev;
  size_t* cap;
};

thread_local std::vector<PinnedSlot> g_slots;

}  // namespace

void track_pinned(void** host, void** dev, size_t* cap) {
  for (const PinnedSlot& s : g_slots)
    if (s.host == host) return;
  g_slots.push_back({host, dev, cap});
}

}  // namespace mpq

// Frees the calling thread's pinned host buffers; the next call that needs one allocates it again.
extern "C" int mpq_release_thread_resources(void) {
  int rc = mpq::kOk;
  if (mpq::g_slots.empty()) return rc;
  // kernels of earlier calls may still write a status mailbox: let the device drain first
  if (hipDeviceSynchronize() != hipSuccess) rc = mpq::kHipError;
  for (const mpq::PinnedSlot& s : mpq::g_slots) {
    if (*s.host && hipHostFree(*s.host) != hipSuccess) rc = mpq::kHipError;
    *s.host = nullptr;
    if (s.dev) *s.dev = nullptr;
    if (s.cap) *s.cap = 0;
  }
  mpq::g_slots.clear();
  if (rc != mpq::kOk) {
    mpq::set_error("mpq_release_thread_resources: a pinned host buffer could not be freed");
    mpq::set_error_code(rc);
  }
  return rc;
}
