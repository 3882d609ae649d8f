// Ticket counters of the prefill kernels' dynamic work tails, handed out per
// stream.
//
// A launch with a dynamic tail (FwdParams::tickets) needs one 32-bit counter
// that is zero when it starts; the workgroup that draws the launch's last
// ticket sets it back to zero, so the next launch on the same stream finds it
// zero again. Launches on one stream run one after another, so each stream
// keeps one counter for all its launches. A launch recorded into a graph may
// later run beside anything else, so it gets a counter of its own for the life
// of the process. The counters are a static per-device array (zero at module
// load), each on its own 128-byte line, whose device address is looked up
// once per device (symbol_address); when they run out, or the stream's
// capture state or device cannot be read, the caller launches without a
// dynamic tail (every work item placed statically), which computes the same
// result.
#include <mutex>
#include <unordered_map>

#include "pf_kernels.hpp"

namespace pf {

namespace {

constexpr int kTicketSlots = 4096;
constexpr int kTicketStride = 32;  // uint32 words per slot (128 bytes)
static __device__ __align__(256) unsigned int ticket_words[kTicketSlots * kTicketStride];

constexpr int kMaxTicketDevices = 64;

struct TicketSlots {
  bool resolved = false;  // address looked up (base == nullptr: unavailable)
  unsigned int* base = nullptr;
  std::mutex mu;
  std::unordered_map<hipStream_t, int> by_stream;
  int used = 0;
};
TicketSlots g_slots[kMaxTicketDevices];

}  // namespace

unsigned int* work_tickets(hipStream_t stream) {
  // The counter must live on the device the launch runs on: the stream's
  // (the null stream's is the current device).
  int dev = -1;
  if (hipStreamGetDevice(stream, &dev) != hipSuccess || dev < 0 || dev >= kMaxTicketDevices) return nullptr;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cs) != hipSuccess) return nullptr;
  TicketSlots& s = g_slots[dev];
  std::lock_guard<std::mutex> lock(s.mu);
  if (!s.resolved) {
    s.resolved = true;
    void* base = nullptr;
    if (symbol_address(dev, HIP_SYMBOL(ticket_words), &base) == hipSuccess) s.base = static_cast<unsigned int*>(base);
  }
  if (s.base == nullptr) return nullptr;
  int slot = -1;
  if (cs == hipStreamCaptureStatusNone) {
    const auto it = s.by_stream.find(stream);
    if (it != s.by_stream.end()) {
      slot = it->second;
    } else if (s.used < kTicketSlots) {
      slot = s.used++;
      s.by_stream.emplace(stream, slot);
    }
  } else if (s.used < kTicketSlots) {
    slot = s.used++;
  }
  return slot < 0 ? nullptr : s.base + (size_t)slot * kTicketStride;
}

}  // namespace pf
