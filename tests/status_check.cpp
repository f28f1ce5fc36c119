// CPU check of the non-finite report's host bookkeeping
// (fe2o3_amd/csrc/status_track.hpp, what fe2o3_rt_stream_synchronize and
// fe2o3_rt_device_synchronize run on the counter they read).  Test
// infrastructure: built with sanitizers and run by
// tests/test_sanitized_host.py.
//   1. A counter that has not moved reports nothing, however often it is read.
//   2. Each change is reported exactly once, by the first read that sees it.
//   3. A mark that lands between two reads is reported by the second: no
//      read clears anything, so no mark can be lost between read and clear.
//   4. Devices are independent.
//   5. Wrap-around of the 32-bit counter still reports.
//   6. Several marks between two reads are one report.
#include <stdint.h>
#include <stdio.h>

#include "../fe2o3_amd/csrc/status_track.hpp"

static int failures = 0;
static void expect(bool ok, const char* what) {
  if (!ok) {
    printf("FAIL %s\n", what);
    ++failures;
  }
}

int main() {
  using fe2o3_host::StatusTracker;
  {
    StatusTracker t;
    expect(!t.report(0), "fresh counter at 0 reports nothing");
    expect(!t.report(0), "unchanged counter reports nothing");
  }
  {
    StatusTracker t;
    expect(t.report(1), "first mark reported");
    expect(!t.report(1), "first mark reported once");
    expect(!t.report(1), "first mark reported once (again)");
    expect(t.report(2), "second mark reported");
    expect(!t.report(2), "second mark reported once");
  }
  {
    // stream A reads 0; a kernel on stream B marks; A's next read sees it.
    // The former read-then-clear could lose a mark landing between the read
    // and the clear; here the device word is only ever added to.
    uint32_t device_counter = 0;
    StatusTracker t;
    expect(!t.report(device_counter), "clean read");
    device_counter += 1;  // mark lands after the read
    expect(t.report(device_counter), "mark after a read is reported by the next read");
    expect(!t.report(device_counter), "and only once");
  }
  {
    StatusTracker d0, d1;
    expect(d0.report(3), "device 0 marks");
    expect(!d1.report(0), "device 1 unaffected");
    expect(d1.report(1), "device 1 marks");
    expect(!d0.report(3), "device 0 unaffected by device 1");
  }
  {
    StatusTracker t;
    expect(t.report(0xffffffffu), "near wrap");
    expect(t.report(0u), "wrap to 0 is a change");
    expect(t.report(5u), "past wrap");
  }
  {
    StatusTracker t;
    expect(t.report(1000u), "many marks between reads are one report");
    expect(!t.report(1000u), "then none");
  }
  printf("failures %d\n", failures);
  return failures == 0 ? 0 : 1;
}
