// status_track.hpp -- host-side bookkeeping of the non-finite report (plain
// C++, no HIP, so a CPU test can build it with g++).
//
// Each device has one 32-bit rejection counter in device memory.  Kernels
// that admit only finite inputs add 1 to it (a relaxed atomic add from one
// lane per rejecting wave or thread) and never clear it; the host never
// writes it either.  A synchronize copies the counter to the host after the
// stream or device has drained and compares it with the count it last
// reported for that device: a different value means at least one rejection
// landed since, and the synchronize reports FE2O3_ERR_NONFINITE.
//
// Nothing is read-then-cleared, so a mark that lands while a synchronize is
// reading is never lost: it is either in the value read or in a later one.
// The counter wraps modulo 2^32; only exactly 2^32 marks between two reports
// would go unseen.  The report is per device and is delivered once, to the
// first synchronize (of any stream of the device, or of the device) whose
// read sees the new count.
#pragma once

#include <stdint.h>

namespace fe2o3_host {

struct StatusTracker {
  uint32_t seen = 0;  // the device counter starts at 0 when the library loads
  // `count`: the counter as just read.  True when rejections arrived since
  // the last report; the count is then taken as reported.
  bool report(uint32_t count) {
    const bool grew = count != seen;
    seen = count;
    return grew;
  }
};

}  // namespace fe2o3_host
