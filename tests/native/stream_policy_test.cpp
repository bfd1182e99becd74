// stream_policy_test.cpp -- GPU-free tests of vx_amd/csrc/vx_stream_policy.h:
// what a wait and a free do for each caller-stream / capture state. The
// table is the one reference runtime/vx_stream_policy.h:23-58 fixes (and
// reference tests/runtime/kernel_launch_test.cpp checks): every row here is
// an outcome a program can observe through the ABI.

#include "../../vx_amd/csrc/vx_stream_policy.h"

#include <cstdio>

namespace {

int failures = 0;

void check(bool ok, const char *what) {
  if (!ok) {
    fprintf(stderr, "FAIL: %s\n", what);
    ++failures;
  }
}

} // namespace

int main() {
  using vx::FreeAction;
  using vx::WaitAction;
  // No caller stream: a wait covers the devices, capture cannot be asked.
  check(vx::wait_action(false, false) == WaitAction::kDevice, "wait, no stream");
  check(vx::wait_action(false, true) == WaitAction::kDevice,
        "wait, no stream (capture is a property of a stream)");
  check(vx::wait_action(true, false) == WaitAction::kStream, "wait, stream");
  check(vx::wait_action(true, true) == WaitAction::kRefuse,
        "wait, capturing stream is refused");

  // Memory from hipMallocAsync goes back in stream order whatever is set now.
  for (int s = 0; s < 2; ++s) {
    for (int c = 0; c < 2; ++c) {
      check(vx::free_action(s, c, true) == FreeAction::kOnStream,
            "stream-ordered memory frees on its stream");
    }
  }
  check(vx::free_action(false, false, false) == FreeAction::kAfterDeviceWait,
        "free, no stream");
  check(vx::free_action(true, false, false) == FreeAction::kAfterStreamWait,
        "free, stream");
  check(vx::free_action(true, true, false) == FreeAction::kRefuse,
        "free that needs a wait, capturing: refused");
  if (failures) {
    fprintf(stderr, "%d failure(s)\n", failures);
    return 1;
  }
  printf("ok\n");
  return 0;
}
